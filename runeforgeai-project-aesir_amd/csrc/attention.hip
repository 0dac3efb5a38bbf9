// Split-KV GQA decode attention for gfx950 (the decode path of flash_attention_gqa,
// compute.mojo:1950-2015).
//
// Grid (split, kv_head). A 256-thread workgroup owns one KV head, all G = nq/nkv query heads that
// share it (so each K/V row is read from HBM once, not G times), and a contiguous chunk of
// positions. K/V tiles of 64 positions are staged in LDS with 16-byte loads (K rows padded by 16
// bytes against bank conflicts); scores use v_dot2_f32_f16; each head's 64 tile scores sit in
// one wave so the tile max/sum are wave reductions; the f32 accumulator is rescaled per tile
// (online softmax). Partials (m, l, acc) go to global memory; the last workgroup of each KV head
// to finish (completion counter, no waiting) merges them and writes f16 outputs.
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

    // ---- write partials (or the final output when this is the only split)
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
    __syncthreads();
    __shared__ int s_last;
    if (tid == 0) s_last = arrive_is_last(a.counters + g, (uint32_t)nsplit) ? 1 : 0;
    __syncthreads();
    if (!s_last) return;
    last_block_acquire();

    // ---- merge: out = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M)
#pragma unroll
    for (int r = 0; r < kMaxPvPasses; r++) {
        const int item = tid + kAThreads * r;
        if (r >= pv_passes || item >= pv_items) continue;
        const int h = item / (hd / 2), d = (item % (hd / 2)) * 2;
        const float *base = a.part + ((int64_t)(g * G + h)) * part_stride;
        float M = -INFINITY;
        for (int64_t s = 0; s < nsplit; s++) M = fmaxf(M, base[s * (hd + 2)]);
        float L = 0.0f, x0 = 0.0f, x1 = 0.0f;
        for (int64_t s = 0; s < nsplit; s++) {
            const float *pp = base + s * (hd + 2);
            const float w = expf(pp[0] - M);
            L = fmaf(pp[1], w, L);
            x0 = fmaf(pp[2 + d], w, x0);
            x1 = fmaf(pp[2 + d + 1], w, x1);
        }
        out[h * hd + d] = (h16)(x0 / L);
        out[h * hd + d + 1] = (h16)(x1 / L);
    }
    if (tid == 0) a.counters[g] = 0;
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
    if (a.max_split < 1 || a.max_split > 65535) return fail(AESIR_ERR_INVALID, "attention: bad split count");
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
    return AESIR_OK;
}

}  // namespace aesir
