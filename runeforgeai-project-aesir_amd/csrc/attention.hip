// Split-KV GQA decode attention for gfx950 (the decode path of flash_attention_gqa,
// compute.mojo:1950-2015).
//
// Grid (split, kv_head). A 256-thread workgroup owns one KV head, all G = nq/nkv query heads that
// share it (so each K/V row is read from HBM once, not G times), and a contiguous chunk of
// positions. K/V tiles of 64 positions are staged in LDS with 16-byte loads (K rows padded by 16
// bytes against bank conflicts); scores use v_dot2_f32_f16; each head's 64 tile scores sit in
// one wave so the tile max/sum are wave reductions; the f32 accumulator is rescaled per tile
// (online softmax). Partials (m, l, acc) go to global memory and a second kernel merges them
// (one workgroup per query head); a single split writes the f16 output directly. No workgroup
// waits on another, and no device-scope fence is needed inside either kernel.
//
// Numerics: the reference rounds its running accumulator to f16 after every position; this
// kernel keeps it in f32 and rounds once at the end (within the 2e-2 / 1e-2 tolerance).
#include <cfloat>

#include "device.hpp"
#include "kernels.hpp"

namespace aesir {

constexpr int kAThreads = 256;
constexpr int kTile = 64;          // positions per LDS tile (one wave of scores per head)
constexpr int kMaxHd = 256;
constexpr int kMaxG = 16;          // query heads per KV head
constexpr int kMaxPvPasses = 8;    // G * hd / 2 <= 256 * kMaxPvPasses
constexpr int kMaxSplit = 128;     // splits per KV head (one merge thread each)
constexpr int kMergeThreads = 128;

int64_t attention_partial_floats(int64_t nq, int64_t hd, int64_t max_split) { return nq * max_split * (hd + 2); }

template <bool VEC>
__global__ __launch_bounds__(kAThreads) void attn_decode_kernel(AttnArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hd = (int)a.hd;
    const int G = (int)(a.nq / a.nkv);
    const int g = blockIdx.y;  // kv head
    const int split = blockIdx.x;
    const int kpad = hd + 8;   // K tile row stride in halves (16-byte pad)

    int64_t S = a.seq_len;
    if (S <= 0) {
        const int64_t pos = a.state->pos;
        S = pos + 1 < a.max_seq ? pos + 1 : a.max_seq;
    }
    int64_t chunk = (S + a.max_split - 1) / a.max_split;
    chunk = (chunk + kTile - 1) / kTile * kTile;
    const int64_t nsplit = (S + chunk - 1) / chunk;
    if (split >= nsplit) return;  // idle workgroup
    const int64_t p0 = split * chunk;
    const int64_t p1 = p0 + chunk < S ? p0 + chunk : S;

    h16 *Kt = reinterpret_cast<h16 *>(smem_raw);          // [kTile][kpad]
    h16 *Vt = Kt + kTile * kpad;                           // [kTile][hd]
    float *sc = reinterpret_cast<float *>(Vt + kTile * hd); // [G][kTile] scores -> probabilities
    h16 *qs = reinterpret_cast<h16 *>(sc + G * kTile);     // [G][hd]
    float *alpha = reinterpret_cast<float *>(qs + G * hd); // [G] per-tile rescale factors

    const h16 *qg = reinterpret_cast<const h16 *>(a.q) + (int64_t)g * G * hd;
    for (int i = tid; i < G * hd; i += kAThreads) qs[i] = qg[i];

    const h16 *Kg = reinterpret_cast<const h16 *>(a.k) + (int64_t)g * hd;
    const h16 *Vg = reinterpret_cast<const h16 *>(a.v) + (int64_t)g * hd;

    // score work: item = tid + 256 * r  ->  head = item / 64, position = item % 64 (= lane)
    const int score_passes = (G * kTile + kAThreads - 1) / kAThreads;
    float m_run[kMaxG / 4], l_run[kMaxG / 4];
#pragma unroll
    for (int r = 0; r < kMaxG / 4; r++) {
        m_run[r] = -INFINITY;
        l_run[r] = 0.0f;
    }
    // PV work: item = tid + 256 * r  ->  head = item / (hd/2), dim pair = item % (hd/2)
    const int pv_items = G * hd / 2;
    const int pv_passes = (pv_items + kAThreads - 1) / kAThreads;
    float acc0[kMaxPvPasses], acc1[kMaxPvPasses];
#pragma unroll
    for (int r = 0; r < kMaxPvPasses; r++) acc0[r] = acc1[r] = 0.0f;

    const int vec_per_row = hd / 8;
    for (int64_t t0 = p0; t0 < p1; t0 += kTile) {
        const int n_here = (int)(p1 - t0 < kTile ? p1 - t0 : kTile);
        __syncthreads();  // previous tile fully consumed
        if (VEC) {
            for (int i = tid; i < n_here * vec_per_row; i += kAThreads) {
                const int p = i / vec_per_row, c = (i % vec_per_row) * 8;
                st16(Kt + p * kpad + c, ld16(Kg + (t0 + p) * a.k_stride + c));
                st16(Vt + p * hd + c, ld16(Vg + (t0 + p) * a.v_stride + c));
            }
        } else {
            for (int i = tid; i < n_here * hd; i += kAThreads) {
                const int p = i / hd, c = i % hd;
                Kt[p * kpad + c] = Kg[(t0 + p) * a.k_stride + c];
                Vt[p * hd + c] = Vg[(t0 + p) * a.v_stride + c];
            }
        }
        __syncthreads();

        // scores and online-softmax bookkeeping; each head's 64 scores live in one wave
#pragma unroll
        for (int r = 0; r < kMaxG / 4; r++) {
            const int item = tid + kAThreads * r;
            const int h = item / kTile, p = item % kTile;
            if (r >= score_passes || h >= G) continue;  // uniform per wave
            float s = -INFINITY;
            if (p < n_here) {
                float d = 0.0f;
                const h16 *kr = Kt + p * kpad;
                const h16 *qr = qs + h * hd;
                if (VEC) {
                    for (int c = 0; c < hd; c += 8) d = dot8(ld16(kr + c), ld16(qr + c), d);
                } else {
                    for (int c = 0; c < hd; c++) d = fmaf((float)kr[c], (float)qr[c], d);
                }
                s = d * a.scale;
            }
            const float tmax = wave_max(s);
            const float m_new = fmaxf(m_run[r], tmax);
            const float pr = p < n_here ? expf(s - m_new) : 0.0f;
            const float tsum = wave_sum(pr);
            const float al = expf(m_run[r] - m_new);
            l_run[r] = l_run[r] * al + tsum;
            m_run[r] = m_new;
            sc[h * kTile + p] = pr;
            if (lane == 0) alpha[h] = al;
        }
        __syncthreads();

#pragma unroll
        for (int r = 0; r < kMaxPvPasses; r++) {
            const int item = tid + kAThreads * r;
            if (r >= pv_passes || item >= pv_items) continue;
            const int h = item / (hd / 2), d = (item % (hd / 2)) * 2;
            const float al = alpha[h];
            float x0 = acc0[r] * al, x1 = acc1[r] * al;
            const float *ph = sc + h * kTile;
            for (int p = 0; p < n_here; p++) {
                const float w = ph[p];
                const h16x2 v = *reinterpret_cast<const h16x2 *>(Vt + p * hd + d);
                x0 = fmaf(w, (float)v.x, x0);
                x1 = fmaf(w, (float)v.y, x1);
            }
            acc0[r] = x0;
            acc1[r] = x1;
        }
    }

    // ---- write partials (or the final output when this is the only split); partial rows are
    // [m, l, acc[hd]] with acc unnormalized, merged by attn_merge_kernel
    const int64_t part_stride = a.max_split * (hd + 2);
    float *mlbuf = reinterpret_cast<float *>(smem_raw);  // reuse LDS: [G] m, [G] l
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kMaxG / 4; r++) {
        const int item = tid + kAThreads * r;
        const int h = item / kTile;
        if (r < score_passes && h < G && lane == 0) {
            mlbuf[h] = m_run[r];
            mlbuf[G + h] = l_run[r];
        }
    }
    __syncthreads();
    h16 *out = reinterpret_cast<h16 *>(a.out) + (int64_t)g * G * hd;
    if (nsplit == 1) {
#pragma unroll
        for (int r = 0; r < kMaxPvPasses; r++) {
            const int item = tid + kAThreads * r;
            if (r >= pv_passes || item >= pv_items) continue;
            const int h = item / (hd / 2), d = (item % (hd / 2)) * 2;
            const float L = mlbuf[G + h];
            out[h * hd + d] = (h16)(acc0[r] / L);
            out[h * hd + d + 1] = (h16)(acc1[r] / L);
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < kMaxPvPasses; r++) {
        const int item = tid + kAThreads * r;
        if (r >= pv_passes || item >= pv_items) continue;
        const int h = item / (hd / 2), d = (item % (hd / 2)) * 2;
        float *pp = a.part + ((int64_t)(g * G + h)) * part_stride + split * (hd + 2);
        pp[2 + d] = acc0[r];
        pp[2 + d + 1] = acc1[r];
        if (d == 0) {
            pp[0] = mlbuf[h];
            pp[1] = mlbuf[G + h];
        }
    }
}

// Merge of the split partials: one workgroup per query head, one split per thread for the
// max/sum bookkeeping, then each thread owns a pair of output dims and accumulates over splits
// with 8 independent loads in flight.
__global__ __launch_bounds__(kMergeThreads) void attn_merge_kernel(AttnArgs a) {
    __shared__ float wsh[kMaxSplit];
    __shared__ float red[kMergeThreads / kWave];
    const int tid = threadIdx.x;
    const int hd = (int)a.hd;
    int64_t S = a.seq_len;
    if (S <= 0) {
        const int64_t pos = a.state->pos;
        S = pos + 1 < a.max_seq ? pos + 1 : a.max_seq;
    }
    int64_t chunk = (S + a.max_split - 1) / a.max_split;
    chunk = (chunk + kTile - 1) / kTile * kTile;
    const int nsplit = (int)((S + chunk - 1) / chunk);
    if (nsplit <= 1) return;  // the partial kernel wrote the output directly
    const int h = blockIdx.x;
    const int64_t stride = hd + 2;
    const float *base = a.part + (int64_t)h * a.max_split * stride;
    const float m_s = tid < nsplit ? base[tid * stride] : -INFINITY;
    const float l_s = tid < nsplit ? base[tid * stride + 1] : 0.0f;
    // M = max_s m_s
    float M = wave_max(m_s);
    if ((tid & 63) == 0) red[tid >> 6] = M;
    __syncthreads();
    M = red[0];
#pragma unroll
    for (int w = 1; w < kMergeThreads / kWave; w++) M = fmaxf(M, red[w]);
    __syncthreads();
    const float w_s = tid < nsplit ? expf(m_s - M) : 0.0f;
    if (tid < kMaxSplit) wsh[tid] = w_s;
    const float L = block_sum<kMergeThreads / kWave>(l_s * w_s, red);  // synchronizes wsh too
    h16 *out = reinterpret_cast<h16 *>(a.out) + (int64_t)h * hd;
    for (int d = 2 * tid; d < hd; d += 2 * kMergeThreads) {
        float x0 = 0.0f, x1 = 0.0f;
        int s = 0;
        for (; s + 8 <= nsplit; s += 8) {
            float2 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = *reinterpret_cast<const float2 *>(base + (s + j) * stride + 2 + d);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                x0 = fmaf(v[j].x, wsh[s + j], x0);
                x1 = fmaf(v[j].y, wsh[s + j], x1);
            }
        }
        for (; s < nsplit; s++) {
            const float2 v = *reinterpret_cast<const float2 *>(base + s * stride + 2 + d);
            x0 = fmaf(v.x, wsh[s], x0);
            x1 = fmaf(v.y, wsh[s], x1);
        }
        out[d] = (h16)(x0 / L);
        out[d + 1] = (h16)(x1 / L);
    }
}

// ------------------------------------------------------------------ fast path (head_dim 64 / 128)
//
// Partial kernel, grid (split, kv_head, head_group). A workgroup owns GH query heads of one KV
// head and every nsplit-th 64-position round of the view (one round for S <= 64 * max_split). All K and V
// requests of a round are issued together before any of them is used, so a round costs one HBM
// round trip:
//   scores   thread t holds dims [16c, 16c + 16) (c = t % TPP) of K rows t / TPP (+ 256 / TPP)
//            and the matching q slices of its GH heads; fdot2 partials are reduced over the TPP
//            lanes of a row, one score per (head, position) lands in LDS
//   V        16-byte loads into LDS, one 256-byte row slice per position
//   softmax  wave h owns head h: one position per lane, round max and sum are wave reductions,
//            the running max / sum stay in that wave's registers (f32 online softmax across
//            rounds), probabilities go back to LDS
//   P V      thread t owns one (head, dim pair) and accumulates over the round from LDS
// The next round's K/V requests are issued before the current round is consumed.
// Each split writes [m, l, acc[HD]] (f32, acc unnormalized); with a single split the kernel
// writes the f16 output itself. attn_fast_merge_kernel (one workgroup per query head) merges.
constexpr int kRound = 64;           // positions per round (one softmax lane each)
constexpr int kMaxFastSplit = 2048;  // splits per KV head of the fast path

// S of a decode launch: the view length, or min(pos + 1, max_seq) from the device state.
__device__ __forceinline__ int64_t decode_seq_len(const AttnArgs &a) {
    if (a.seq_len > 0) return a.seq_len;
    const int64_t pos = a.state->pos;
    return pos + 1 < a.max_seq ? pos + 1 : a.max_seq;
}

// Splits of S positions: each covers at most ceil(rounds / max_split) 64-position rounds, so
// nsplit = ceil(rounds / per) with per = ceil(rounds / max_split) (the same as whole-round chunks
// of ceil(S / max_split) positions, by ceil(ceil(a / b) / c) = ceil(a / (b c))). 32-bit divisions:
// a 64-bit one is a long dependent sequence at the head of both kernels.
__device__ __forceinline__ int split_count(int64_t S, int64_t max_split) {
    const uint32_t rounds = (uint32_t)((S + kRound - 1) / kRound), ms = (uint32_t)max_split;
    const uint32_t per = (rounds + ms - 1) / ms;
    return (int)((rounds + per - 1) / per);
}

// NG > 1 (short views, one split): NG groups of 256 threads share the workgroup; group q takes
// rounds q, q + NG, ... of the view (every group runs the same number of loop iterations, the
// surplus ones masked), and the groups' (m, l, acc) are combined in LDS before the output is
// written, so no merge launch follows.
template <int HD, int GH, int NG>
__global__ __launch_bounds__(kAThreads * NG) void attn_fast_kernel(AttnArgs a) {
    constexpr int TPP = HD / 16;              // score threads per K row (16 dims each)
    constexpr int RPP = kAThreads / TPP;      // K rows per score pass
    constexpr int NSP = kRound / RPP;         // score passes per round (2 for HD 128, 1 for HD 64)
    constexpr int VCH = HD / 8;               // 16-byte chunks per V row slice
    constexpr int NVL = kRound * VCH / kAThreads;  // V loads per thread per round
    constexpr int kItems = GH * HD / 2;       // PV items: (head, dim pair)
    constexpr int PVS = kAThreads / kItems;   // PV position groups (1, 2, 4 or 8)
    constexpr int NPOS = kRound / PVS;        // positions per thread per round in the PV pass
    static_assert(NSP * RPP == kRound && NVL * kAThreads == kRound * VCH && kItems * PVS == kAThreads, "shape");
    __shared__ __align__(16) float scs[NG][GH][kRound];  // scores, then probabilities
    __shared__ __align__(16) h16 vss[NG][kRound][HD];
    __shared__ float alphas[NG][GH], mruns[NG][GH], lruns[NG][GH];
    __shared__ float2 pvxs[NG][PVS > 1 ? PVS - 1 : 1][kItems];
    __shared__ float2 gacc[NG > 1 ? NG - 1 : 1][kItems];

    const int tid = threadIdx.x % kAThreads, grp = threadIdx.x / kAThreads;  // thread in its group
    const int lane = tid & 63, wave = tid >> 6;
    auto &sc = scs[grp];
    auto &vs = vss[grp];
    auto &alpha = alphas[grp];
    auto &mrun = mruns[grp];
    auto &lrun = lruns[grp];
    auto &pvx = pvxs[grp];
    const int64_t G = (int64_t)GH * gridDim.z;  // query heads per KV head (the grid's z is G / GH)
    const int g = blockIdx.y, hg = blockIdx.z;
    const int split = blockIdx.x;
    const int64_t S = decode_seq_len(a);
    const int nsplit = split_count(S, a.max_split);
    if (split >= nsplit) return;  // idle workgroup
    // Split s takes the rounds s, s + nsplit, s + 2 nsplit, ... of the view (rounds dealt out, not
    // a contiguous chunk): at each step the splits together read one contiguous stretch of rows,
    // so the grid sweeps the cache front to back (KV 32768 at the Llama-3 shape: 31.7 -> 28.0 us
    // per layer for the partials) and a split's partial still covers ceil(rounds / max_split)
    // rounds at most.
    const int64_t p0 = (int64_t)split * kRound;
    const int64_t p1 = S;
    const int64_t head0 = (int64_t)g * G + (int64_t)hg * GH;  // first query head of this workgroup

    const int sp = tid / TPP, sc_c = tid % TPP;                  // score row / dim chunk
    const int item = tid % kItems, pg = tid / kItems;            // PV item / position group
    const int ph = item / (HD / 2), pd = (item % (HD / 2)) * 2;  // PV head / dim pair
    const h16 *Kb = reinterpret_cast<const h16 *>(a.k) + (int64_t)g * HD + 16 * sc_c;
    const h16 *Vb = reinterpret_cast<const h16 *>(a.v) + (int64_t)g * HD;

    // K/V requests of one round (rows past p1 re-read row t0 and are masked)
    auto load_round = [&](int64_t t0, u32x4 (&kr)[NSP][2], u32x4 (&vr)[NVL]) {
        if constexpr (NG > 1)
            if (t0 >= p1) t0 = p0;  // a group's surplus round re-reads the first round (masked)
        const int n = (int)(p1 - t0 < kRound ? p1 - t0 : kRound);
#pragma unroll
        for (int i = 0; i < NSP; i++) {
            const int r = sp + i * RPP;
            const int64_t p = t0 + (r < n ? r : 0);
            kr[i][0] = ld16(Kb + p * a.k_stride);
            kr[i][1] = ld16(Kb + p * a.k_stride + 8);
        }
#pragma unroll
        for (int i = 0; i < NVL; i++) {
            const int e = tid + i * kAThreads, r = e / VCH, c = e % VCH;
            vr[i] = ld16(Vb + (t0 + (r < n ? r : 0)) * a.v_stride + 8 * c);
        }
    };
    const int nrounds = (int)((p1 - p0 + kRound - 1) / kRound);
    const int iters = (nrounds + NG - 1) / NG;  // loop iterations of every group
    auto round_t0 = [&](int j) { return p0 + (int64_t)kRound * (grp + NG * j); };
    u32x4 kr[NSP][2], vr[NVL], kn[NSP][2], vn[NVL];
    load_round(NG > 1 ? round_t0(0) : p0, kr, vr);
    u32x4 qr[GH][2];
    {
        const h16 *qb = reinterpret_cast<const h16 *>(a.q) + head0 * HD + 16 * sc_c;
#pragma unroll
        for (int h = 0; h < GH; h++) {
            qr[h][0] = ld16(qb + h * HD);
            qr[h][1] = ld16(qb + h * HD + 8);
        }
    }
    float m_w = -INFINITY, l_w = 0.0f;  // running softmax state of head `wave` (waves < GH)
    float acc0 = 0.0f, acc1 = 0.0f;
    // One round: scores, V to LDS, online softmax, P V. The caller owns the barrier that lets the
    // next round rewrite sc and vs.
    auto round = [&](int64_t t0, const u32x4 (&kc)[NSP][2], const u32x4 (&vc)[NVL]) {
        const int n_here = NG > 1 && t0 >= p1 ? 0 : (int)(p1 - t0 < kRound ? p1 - t0 : kRound);  // 0: surplus round
#pragma unroll
        for (int i = 0; i < NSP; i++) {
#pragma unroll
            for (int h = 0; h < GH; h++) {
                float d = dot8(kc[i][0], qr[h][0], 0.0f);
                d = dot8(kc[i][1], qr[h][1], d);
                d = group_sum<TPP>(d);
                if (sc_c == 0) sc[h][sp + i * RPP] = d * a.scale;
            }
        }
#pragma unroll
        for (int i = 0; i < NVL; i++) {
            const int e = tid + i * kAThreads, r = e / VCH, c = e % VCH;
            st16(&vs[r][8 * c], vc[i]);
        }
        __syncthreads();
        // online softmax of head `wave` over the round (one position per lane)
        if (wave < GH && (NG == 1 || n_here > 0)) {
            const float s = lane < n_here ? sc[wave][lane] : -INFINITY;
            const float mn = fmaxf(m_w, wave_max(s));
            const float pr = lane < n_here ? expf(s - mn) : 0.0f;
            const float al = expf(m_w - mn);  // 0 on the first round (m_w = -inf)
            l_w = l_w * al + wave_sum(pr);
            m_w = mn;
            sc[wave][lane] = pr;
            if (lane == 0) alpha[wave] = al;
        }
        __syncthreads();
        // P V over this thread's positions of the round (probabilities are 0 beyond n_here)
        if (NG > 1 && n_here == 0) return;
        const float al = alpha[ph];
        acc0 *= al;
        acc1 *= al;
#pragma unroll
        for (int j = 0; j < NPOS; j += 4) {
            const f32x4 w = *reinterpret_cast<const f32x4 *>(&sc[ph][pg * NPOS + j]);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const h16x2 v = *reinterpret_cast<const h16x2 *>(&vs[pg * NPOS + j + u][pd]);
                acc0 = fmaf(w[u], (float)v.x, acc0);
                acc1 = fmaf(w[u], (float)v.y, acc1);
            }
        }
    };
    // Rounds with a successor request it before computing (unconditionally, so the compiler's wait
    // counts stay exact and the successor's loads overlap this round); the last round follows.
    if constexpr (NG == 1) {
        const int64_t step = (int64_t)nsplit * kRound;
        int64_t t0 = p0;
        for (; t0 + step < p1; t0 += step) {
            load_round(t0 + step, kn, vn);
            round(t0, kr, vr);
#pragma unroll
            for (int i = 0; i < NSP; i++) {
                kr[i][0] = kn[i][0];
                kr[i][1] = kn[i][1];
            }
#pragma unroll
            for (int i = 0; i < NVL; i++) vr[i] = vn[i];
            __syncthreads();  // sc and vs are rewritten by the next round
        }
        round(t0, kr, vr);
    } else {
        int j = 0;
        for (; j + 1 < iters; j++) {
            load_round(round_t0(j + 1), kn, vn);
            round(round_t0(j), kr, vr);
#pragma unroll
            for (int i = 0; i < NSP; i++) {
                kr[i][0] = kn[i][0];
                kr[i][1] = kn[i][1];
            }
#pragma unroll
            for (int i = 0; i < NVL; i++) vr[i] = vn[i];
            __syncthreads();
        }
        round(round_t0(j), kr, vr);
    }

    if constexpr (NG > 1) {  // combine the groups (one split: the output is written here)
        if (wave < GH && lane == 0) {
            mrun[wave] = m_w;
            lrun[wave] = l_w;
        }
        if (PVS > 1 && pg > 0) pvx[pg - 1][item] = float2{acc0, acc1};
        __syncthreads();
        if (pg == 0) {
#pragma unroll
            for (int q = 0; q < PVS - 1; q++) {
                const float2 o = pvx[q][item];
                acc0 += o.x;
                acc1 += o.y;
            }
            if (grp > 0) gacc[grp - 1][item] = float2{acc0, acc1};
        }
        __syncthreads();
        if (grp == 0 && pg == 0) {
            float M = mruns[0][ph];
#pragma unroll
            for (int q = 1; q < NG; q++) M = fmaxf(M, mruns[q][ph]);  // group 0 always has a round
            float L = lruns[0][ph] * expf(mruns[0][ph] - M);
            acc0 *= expf(mruns[0][ph] - M);
            acc1 *= expf(mruns[0][ph] - M);
#pragma unroll
            for (int q = 1; q < NG; q++) {
                const float e = expf(mruns[q][ph] - M);  // 0 for a group without rounds
                const float2 o = gacc[q - 1][item];
                L = fmaf(lruns[q][ph], e, L);
                acc0 = fmaf(o.x, e, acc0);
                acc1 = fmaf(o.y, e, acc1);
            }
            h16 *out = reinterpret_cast<h16 *>(a.out) + (head0 + ph) * HD + pd;
            out[0] = (h16)(acc0 / L);
            out[1] = (h16)(acc1 / L);
        }
        return;
    }

    // Write the partial (or the output for one split). With one PV position group and one head
    // per wave (head_dim 128, 4 heads per workgroup), thread t's head is its wave's, whose
    // running max and sum are already in its registers.
    if constexpr (PVS == 1 && HD / 2 == kWave && GH == kAThreads / kWave) {
        if (nsplit == 1) {
            h16 *out = reinterpret_cast<h16 *>(a.out) + (head0 + ph) * HD + pd;
            out[0] = (h16)(acc0 / l_w);
            out[1] = (h16)(acc1 / l_w);
        } else {
            float *pp = a.part + ((head0 + ph) * a.max_split + split) * (HD + 2);
            *reinterpret_cast<float2 *>(pp + 2 + pd) = float2{acc0, acc1};
            if (pd == 0) *reinterpret_cast<float2 *>(pp) = float2{m_w, l_w};
        }
        return;
    }
    // otherwise combine the PV position groups through LDS first
    if (wave < GH && lane == 0) {
        mrun[wave] = m_w;
        lrun[wave] = l_w;
    }
    if (PVS > 1 && pg > 0) pvx[pg - 1][item] = float2{acc0, acc1};
    __syncthreads();
    if (pg != 0) return;
#pragma unroll
    for (int j = 0; j < PVS - 1; j++) {
        const float2 o = pvx[j][item];
        acc0 += o.x;
        acc1 += o.y;
    }
    if (nsplit == 1) {
        h16 *out = reinterpret_cast<h16 *>(a.out) + (head0 + ph) * HD + pd;
        out[0] = (h16)(acc0 / lrun[ph]);
        out[1] = (h16)(acc1 / lrun[ph]);
    } else {
        float *pp = a.part + ((head0 + ph) * a.max_split + split) * (HD + 2);
        *reinterpret_cast<float2 *>(pp + 2 + pd) = float2{acc0, acc1};
        if (pd == 0) *reinterpret_cast<float2 *>(pp) = float2{mrun[ph], lrun[ph]};
    }
}

// Merge of the split partials, one workgroup per query head: w_s = exp(m_s - max m),
// out = f16(sum_s w_s acc_s / sum_s w_s l_s). Thread t owns dim pair t % (HD/2) over the splits
// s = t / (HD/2) (mod NG). The (m, l) pair of split t and the accumulators of the first 64
// splits (the decode step's maximum) are requested together, so a merge costs one round trip.
template <int HD>
__global__ __launch_bounds__(kAThreads) void attn_fast_merge_kernel(AttnArgs a) {
    constexpr int NDP = HD / 2;
    constexpr int NG = kAThreads / NDP;
    constexpr int kPre = 64 / NG;
    constexpr int kW = kAThreads / kWave;
    __shared__ float wsh[kMaxFastSplit];
    __shared__ float redm[kW], reds[kW];
    __shared__ float2 gx[NG][NDP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t S = decode_seq_len(a);
    const int nsplit = split_count(S, a.max_split);
    if (nsplit <= 1) return;  // the partial kernel wrote the output
    const int64_t h = blockIdx.x;
    const float *base = a.part + h * a.max_split * (HD + 2);
    const int dp = tid % NDP, sg = tid / NDP;

    const float2 ml = tid < nsplit ? *reinterpret_cast<const float2 *>(base + (int64_t)tid * (HD + 2))
                                   : float2{-INFINITY, 0.0f};
    float2 pre[kPre];
#pragma unroll
    for (int j = 0; j < kPre; j++) {
        const int s = sg + NG * j;
        pre[j] = s < nsplit ? *reinterpret_cast<const float2 *>(base + (int64_t)s * (HD + 2) + 2 + 2 * dp)
                            : float2{0.0f, 0.0f};
    }
    float mloc = ml.x;
    for (int s = tid + kAThreads; s < nsplit; s += kAThreads) mloc = fmaxf(mloc, base[(int64_t)s * (HD + 2)]);
    mloc = wave_max(mloc);
    if (lane == 0) redm[wave] = mloc;
    __syncthreads();
    float M = redm[0];
#pragma unroll
    for (int w = 1; w < kW; w++) M = fmaxf(M, redm[w]);
    float lsum = 0.0f;
    if (tid < nsplit) {
        const float e = expf(ml.x - M);
        wsh[tid] = e;
        lsum = ml.y * e;
    }
    for (int s = tid + kAThreads; s < nsplit; s += kAThreads) {
        const float2 m2 = *reinterpret_cast<const float2 *>(base + (int64_t)s * (HD + 2));
        const float e = expf(m2.x - M);
        wsh[s] = e;
        lsum = fmaf(m2.y, e, lsum);
    }
    lsum = wave_sum(lsum);
    if (lane == 0) reds[wave] = lsum;
    __syncthreads();  // also publishes wsh
    float L = reds[0];
#pragma unroll
    for (int w = 1; w < kW; w++) L += reds[w];
    float x0 = 0.0f, x1 = 0.0f;
#pragma unroll
    for (int j = 0; j < kPre; j++) {
        const int s = sg + NG * j;
        if (s < nsplit) {
            x0 = fmaf(pre[j].x, wsh[s], x0);
            x1 = fmaf(pre[j].y, wsh[s], x1);
        }
    }
    for (int s0 = sg + NG * kPre; s0 < nsplit; s0 += NG * kPre) {  // more than 64 splits: kPre loads per batch
        float2 v[kPre];
#pragma unroll
        for (int j = 0; j < kPre; j++) {
            const int s = s0 + NG * j;
            v[j] = s < nsplit ? *reinterpret_cast<const float2 *>(base + (int64_t)s * (HD + 2) + 2 + 2 * dp)
                              : float2{0.0f, 0.0f};
        }
#pragma unroll
        for (int j = 0; j < kPre; j++) {
            const int s = s0 + NG * j;
            if (s < nsplit) {
                x0 = fmaf(v[j].x, wsh[s], x0);
                x1 = fmaf(v[j].y, wsh[s], x1);
            }
        }
    }
    gx[sg][dp] = float2{x0, x1};
    __syncthreads();
    if (sg != 0) return;
#pragma unroll
    for (int j = 1; j < NG; j++) {
        x0 += gx[j][dp].x;
        x1 += gx[j][dp].y;
    }
    h16 *out = reinterpret_cast<h16 *>(a.out) + h * HD + 2 * dp;
    out[0] = (h16)(x0 / L);
    out[1] = (h16)(x1 / L);
}

// Query heads per workgroup of the fast path (0: the generic kernels serve this shape).
static int fast_group(const AttnArgs &a) {
    const int64_t G = a.nq / a.nkv;
    if (a.hd != 64 && a.hd != 128) return 0;
    if (a.max_split > kMaxFastSplit) return 0;
    if (a.k_stride % 8 != 0 || a.v_stride % 8 != 0) return 0;
    if (((uintptr_t)a.k & 15) || ((uintptr_t)a.v & 15) || ((uintptr_t)a.q & 15)) return 0;
    // few splits (short views of a multi-split plan): 2 heads per workgroup give twice the
    // workgroups (Llama-3 shape at KV 512, 9 splits x 8 KV heads: attention 7.4-7.5 -> 7.0 us)
    if (a.max_split > 1 && a.max_split * a.nkv < 128 && G % 2 == 0) return 2;
    return G % 4 == 0 ? 4 : G % 2 == 0 ? 2 : 1;
}

// Views of at most this many positions run as one split: one workgroup per head group with
// kSingleGroups(hd) groups of 256 threads taking two rounds each at most, and no merge launch.
static int64_t single_split_max(int64_t hd) { return hd == 64 ? 8 * kRound : hd == 128 ? 4 * kRound : 0; }

// Split count: one split for short views (above); otherwise one 64-position round per split up
// to 64 splits (more splits cost more in the merge than they gain in parallelism on MI355X;
// longer views give each split several rounds).
int64_t attention_split_count(int64_t hd, int64_t max_positions) {
    if (max_positions <= single_split_max(hd)) return 1;
    const bool fast = hd == 64 || hd == 128;
    const int64_t per = fast ? kRound : kTile;
    const int64_t cap = fast ? 64 : kMaxSplit;
    int64_t n = (max_positions + per - 1) / per;
    if (n > cap) n = cap;
    return n < 1 ? 1 : n;
}

static int64_t attn_lds_bytes(int64_t G, int64_t hd) {
    return (int64_t)kTile * (hd + 8) * 2 + (int64_t)kTile * hd * 2 + G * kTile * 4 + G * hd * 2 + G * 4 + 64;
}

int32_t launch_attention_decode(hipStream_t s, const AttnArgs &a) {
    const int64_t G = a.nq / a.nkv;
    if (a.hd > kMaxHd || a.hd % 2 != 0)
        return fail(AESIR_ERR_UNSUPPORTED, "attention: head_dim %lld not supported (even, <= %d)", (long long)a.hd, kMaxHd);
    if (G > kMaxG) return fail(AESIR_ERR_UNSUPPORTED, "attention: %lld query heads per KV head exceeds %d", (long long)G, kMaxG);
    if (G * a.hd / 2 > (int64_t)kAThreads * kMaxPvPasses)
        return fail(AESIR_ERR_UNSUPPORTED, "attention: query group x head_dim too large");
    if (a.max_split < 1 || a.max_split > kMaxFastSplit) return fail(AESIR_ERR_INVALID, "attention: bad split count");
    if (a.hd / 2 > kMergeThreads * 64) return fail(AESIR_ERR_UNSUPPORTED, "attention: head_dim too large for the merge");
    if (const int gh = fast_group(a); gh && a.max_split == 1) {
        // one split: NG groups per workgroup (4 for head_dim 64 with one head per workgroup, 2
        // for head_dim 128 with up to 4, whose registers allow only 2 groups), no merge. One head
        // per workgroup at head_dim 64 doubles the workgroups of a short view (K/V rows are then
        // read once per head, from L2): TinyLlama decode 1612 -> 1635 tok/s against 2 heads.
        const int gs = a.hd == 64 ? 1 : gh;
        const dim3 grid(1u, (unsigned)a.nkv, (unsigned)(G / gs));
#define AESIR_ATTN_ONE(HDV, GHV, NGV)                                                          \
    if (a.hd == HDV && gs == GHV) hipLaunchKernelGGL((attn_fast_kernel<HDV, GHV, NGV>), grid, dim3(kAThreads * NGV), 0, s, a);
        AESIR_ATTN_ONE(128, 4, 2)
        AESIR_ATTN_ONE(128, 2, 2)
        AESIR_ATTN_ONE(128, 1, 2)
        AESIR_ATTN_ONE(64, 2, 4)
        AESIR_ATTN_ONE(64, 1, 4)
#undef AESIR_ATTN_ONE
        AESIR_LAUNCH_CHECK("attn_fast_kernel (one split)");
        return AESIR_OK;
    }
    if (const int gh = fast_group(a)) {
        const dim3 grid((unsigned)a.max_split, (unsigned)a.nkv, (unsigned)(G / gh));
#define AESIR_ATTN_FAST(HDV, GHV)                                                              \
    if (a.hd == HDV && gh == GHV) hipLaunchKernelGGL((attn_fast_kernel<HDV, GHV, 1>), grid, dim3(kAThreads), 0, s, a);
        AESIR_ATTN_FAST(128, 4)
        AESIR_ATTN_FAST(128, 2)
        AESIR_ATTN_FAST(128, 1)
        AESIR_ATTN_FAST(64, 4)
        AESIR_ATTN_FAST(64, 2)
        AESIR_ATTN_FAST(64, 1)
#undef AESIR_ATTN_FAST
        AESIR_LAUNCH_CHECK("attn_fast_kernel");
        if (a.hd == 128)
            hipLaunchKernelGGL(attn_fast_merge_kernel<128>, dim3((unsigned)a.nq), dim3(kAThreads), 0, s, a);
        else
            hipLaunchKernelGGL(attn_fast_merge_kernel<64>, dim3((unsigned)a.nq), dim3(kAThreads), 0, s, a);
        AESIR_LAUNCH_CHECK("attn_fast_merge_kernel");
        return AESIR_OK;
    }
    if (a.max_split > kMaxSplit) return fail(AESIR_ERR_INVALID, "attention: bad split count");
    const bool vec = a.hd % 8 == 0 && a.k_stride % 8 == 0 && a.v_stride % 8 == 0 && ((uintptr_t)a.k & 15) == 0 &&
                     ((uintptr_t)a.v & 15) == 0 && ((uintptr_t)a.q & 15) == 0;
    const int64_t lds = attn_lds_bytes(G, a.hd);
    const dim3 grid((unsigned)a.max_split, (unsigned)a.nkv);
    if (vec) {
        if (lds > 64 * 1024)
            AESIR_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(attn_decode_kernel<true>),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL(attn_decode_kernel<true>, grid, dim3(kAThreads), (unsigned)lds, s, a);
    } else {
        if (lds > 64 * 1024)
            AESIR_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(attn_decode_kernel<false>),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL(attn_decode_kernel<false>, grid, dim3(kAThreads), (unsigned)lds, s, a);
    }
    AESIR_LAUNCH_CHECK("attn_decode_kernel");
    hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)a.nq), dim3(kMergeThreads), 0, s, a);
    AESIR_LAUNCH_CHECK("attn_merge_kernel");
    return AESIR_OK;
}

}  // namespace aesir
