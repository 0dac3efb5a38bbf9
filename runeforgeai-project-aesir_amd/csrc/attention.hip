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
    if (split >= nsplit) return;  // idle workgroup: does not take part in the merge count
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
    if (a.max_split < 1 || a.max_split > kMaxSplit) return fail(AESIR_ERR_INVALID, "attention: bad split count");
    if (a.hd / 2 > kMergeThreads * 64) return fail(AESIR_ERR_UNSUPPORTED, "attention: head_dim too large for the merge");
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
