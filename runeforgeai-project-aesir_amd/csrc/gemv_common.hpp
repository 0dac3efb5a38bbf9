// Pieces shared by the decode GEMV kernels (gemv.hip: F16 and Q8_0 weights; quant.hip: Q4_0,
// Q4_K and Q6_K weights): workgroup shape, the RMSNorm prologue helpers, the row-sum view and
// the fused epilogues.
#pragma once

#include "device.hpp"
#include "kernels.hpp"

namespace aesir {

constexpr int kThreads = 256;

// Row sums of a ROWS-row workgroup: red[w * ROWS + r] holds wave w's sum of row r; each
// epilogue thread adds up the rows it needs (same order for every reader).
template <int ROWS>
struct RowSums {
    const float *red;
    __device__ __forceinline__ float operator[](int r) const {
        return (red[r] + red[ROWS + r]) + (red[2 * ROWS + r] + red[3 * ROWS + r]);
    }
};

__device__ __forceinline__ float sumsq8(u32x4 v, float acc) {
    unsigned w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        h16x2 h = as_h2(w[i]);
        float a = (float)h.x, b = (float)h.y;
        acc = fmaf(a, a, acc);
        acc = fmaf(b, b, acc);
    }
    return acc;
}

// rmsnorm scale of one 8-element chunk: f16(f16(x * inv) * w) per element
// (compute.mojo:2195-2204).
__device__ __forceinline__ u32x4 norm8(u32x4 x, u32x4 w, h16 inv) {
    unsigned xs[4] = {x.x, x.y, x.z, x.w}, ws[4] = {w.x, w.y, w.z, w.w}, o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        h16x2 a = as_h2(xs[i]), b = as_h2(ws[i]), r;
        r.x = hmul(hmul(a.x, inv), b.x);
        r.y = hmul(hmul(a.y, inv), b.y);
        o[i] = h2_bits(r);
    }
    return u32x4{o[0], o[1], o[2], o[3]};
}

// Weight slabs in flight per thread (F16 and Q8_0 kernels). Measured on MI355X, Llama-3-8B shapes:
// 3 or 4 slabs are no faster than 2 on any decode GEMV (the down projection, 7 slabs, stays at
// 19.5-20 us; gate/up 35.2 us becomes 37.3).
constexpr int kGemvDepth = 2;

// ------------------------------------------------------------------ epilogues

// Each epilogue has a prefetch() that the kernels call right after the first weight requests, so
// any operand the epilogue reads from memory arrives with the weights instead of adding a
// dependent round trip at the end of the workgroup.
struct NoPre {};

struct EpiStore {
    h16 *y;
    int64_t ldy;
    template <int ROWS>
    __device__ __forceinline__ NoPre prefetch(int64_t, int64_t, int64_t, int) const { return {}; }
    template <int ROWS, class S>
    __device__ __forceinline__ void apply(int64_t n0, int64_t m, int64_t N, const S &s, int tid, NoPre) const {
        if (tid < ROWS && n0 + tid < N) y[m * ldy + n0 + tid] = (h16)s[tid];
    }
};

// O projection / down projection: x = f16(f16(acc) + x)  (inference.mojo:227-232, 268-273).
struct EpiResidual {
    h16 *x;
    template <int ROWS>
    __device__ __forceinline__ h16 prefetch(int64_t n0, int64_t, int64_t N, int tid) const {
        return (tid < ROWS && n0 + tid < N) ? x[n0 + tid] : (h16)0.0f;  // only this workgroup writes it
    }
    template <int ROWS, class S>
    __device__ __forceinline__ void apply(int64_t n0, int64_t, int64_t N, const S &s, int tid, h16 old) const {
        if (tid < ROWS && n0 + tid < N) x[n0 + tid] = hadd((h16)s[tid], old);
    }
};

// QKV rows: f16 outputs; RoPE on Q and K pairs (apply_rope, compute.mojo:2232-2244) with the
// host-built cos/sin table; K and V written to the cache slot pos % max_seq (KVCache.append,
// mimir_well.mojo:488-501).
struct EpiQkv {
    h16 *q;
    h16 *kc, *vc;
    const h16x2 *rope;
    const DecodeState *state;
    int64_t dim, kvd, hd, max_seq;
    struct Pre {
        int64_t pos, slot;  // position and its cache row (pos % max_seq, taken while the weights stream)
        h16x2 cs;           // cos/sin of this thread's pair (Q and K rows)
    };
    template <int ROWS>
    __device__ __forceinline__ Pre prefetch(int64_t n0, int64_t, int64_t N, int tid) const {
        Pre p{state->pos, 0, h16x2{(h16)1.0f, (h16)0.0f}};
        p.slot = p.pos % max_seq;
        const int64_t n = n0 + 2 * tid;
        if (tid < ROWS / 2 && n < N && n < dim + kvd) {
            const int64_t nn = n < dim ? n : n - dim;
            p.cs = rope[p.pos * (hd / 2) + ((nn % hd) >> 1)];
        }
        return p;
    }
    template <int ROWS, class S>
    __device__ __forceinline__ void apply(int64_t n0, int64_t, int64_t N, const S &s, int tid, const Pre &pre) const {
        static_assert(ROWS % 2 == 0, "pairs must stay in one workgroup");
        if (tid >= ROWS / 2) return;
        const int64_t n = n0 + 2 * tid;
        if (n >= N) return;
        const h16 s0 = (h16)s[2 * tid], s1 = (h16)s[2 * tid + 1];
        const int64_t slot = pre.slot;
        if (n < dim + kvd) {
            const int64_t nn = n < dim ? n : n - dim;
            const h16x2 cs = pre.cs;
            const h16 r0 = hsub(hmul(s0, cs.x), hmul(s1, cs.y));
            const h16 r1 = hadd(hmul(s0, cs.y), hmul(s1, cs.x));
            h16 *dst = n < dim ? q + nn : kc + slot * kvd + nn;
            dst[0] = r0;
            dst[1] = r1;
        } else {
            h16 *dst = vc + slot * kvd + (n - dim - kvd);
            dst[0] = s0;
            dst[1] = s1;
        }
    }
};

// Interleaved gate/up rows: act = f16(f16(up) * silu(f16(gate)))  (inference.mojo:254-260).
struct EpiSwiglu {
    h16 *act;
    template <int ROWS>
    __device__ __forceinline__ NoPre prefetch(int64_t, int64_t, int64_t, int) const { return {}; }
    template <int ROWS, class S>
    __device__ __forceinline__ void apply(int64_t n0, int64_t, int64_t N, const S &s, int tid, NoPre) const {
        if (tid >= ROWS / 2 || n0 + 2 * tid >= N) return;
        const h16 g = (h16)s[2 * tid], u = (h16)s[2 * tid + 1];
        act[n0 / 2 + tid] = hmul(u, silu_h(g));
    }
};

struct ArgPart {
    float v;
    int32_t i;
};

constexpr float kArgmaxFloor = -10000.0f;  // f16(-10000) is exact (inference.mojo:508)

// Combines two scan results where `b` covers higher indices: b wins only if strictly greater,
// which reproduces the reference's ascending scan with strict '>' (inference.mojo:510-514).
__device__ __forceinline__ ArgPart arg_combine(ArgPart a, ArgPart b) { return b.v > a.v ? b : a; }

// Per-group scan of the ROWS logits of one workgroup in ascending order.
template <int ROWS, class S>
__device__ __forceinline__ ArgPart group_scan(int64_t n0, int64_t N, const S &s) {
    float cv = kArgmaxFloor;
    int32_t ci = -1;
    for (int r = 0; r < ROWS && n0 + r < N; r++) {
        float v = (float)(h16)s[r];
        if (v > cv) {
            cv = v;
            ci = (int32_t)(n0 + r);
        }
    }
    return ci >= 0 ? ArgPart{cv, ci} : ArgPart{-INFINITY, -1};
}

// lm_head: f16 logits plus one ordered (value, index) partial per workgroup; argmax_finish_kernel
// reduces the partials in a second launch.
struct EpiLmHead {
    h16 *logits;
    ArgPart *parts;
    template <int ROWS>
    __device__ __forceinline__ NoPre prefetch(int64_t, int64_t, int64_t, int) const { return {}; }
    template <int ROWS, class S>
    __device__ __forceinline__ void apply(int64_t n0, int64_t, int64_t N, const S &s, int tid, NoPre) const {
        if (tid < ROWS && n0 + tid < N) logits[n0 + tid] = (h16)s[tid];
        if (tid == 0 && n0 < N) parts[n0 / ROWS] = group_scan<ROWS>(n0, N, s);
    }
};

// Decode-step GEMVs of Q4_0 / Q4_K / Q6_K matrices with these epilogues (quant.hip).
int32_t launch_qf_qkv_rope_kv(hipStream_t s, const QkvArgs &a, const EpiQkv &e);
int32_t launch_qf_lm_head(hipStream_t s, const LmHeadArgs &a, const EpiLmHead &e);

}  // namespace aesir
