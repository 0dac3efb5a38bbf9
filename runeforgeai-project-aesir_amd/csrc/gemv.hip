// Decode GEMV for gfx950: y = W x with W [N][K] f16 row-major, f32 accumulation, f16 output.
//
// Bandwidth design (HBM-bound, ~1 flop per byte): a 256-thread workgroup owns ROWS consecutive
// rows; every thread streams 16-byte non-temporal loads of those rows at its k offsets
// (k = 8*tid + 2048*i), so each wave reads contiguous 1 KiB segments. x is staged once per
// workgroup in LDS (optionally RMS-normalized on the way in, which fuses rmsnorm into the
// consumer of its output). Products use v_dot2_f32_f16; the per-row partials are reduced with a
// recursive-halving wave reduction (ROWS rows in log2(64) steps) and one LDS exchange across the
// four waves. The epilogue functor receives the ROWS f32 sums and applies the fused tail: f16
// store, residual add, RoPE + KV append, SwiGLU, or logits + argmax.
#include <cfloat>

#include "device.hpp"
#include "gemv_common.hpp"
#include "kernels.hpp"

namespace aesir {

constexpr int kSlab = kThreads * 8;  // k elements covered by one pass of the workgroup

__device__ __forceinline__ u32x4 gather8(const h16 *p, int64_t k, int64_t K) {
    uint16_t t[8];
#pragma unroll
    for (int j = 0; j < 8; j++) t[j] = (k + j < K) ? h_to_bits(p[k + j]) : (uint16_t)0;
    u32x4 v;
    v.x = t[0] | ((unsigned)t[1] << 16);
    v.y = t[2] | ((unsigned)t[3] << 16);
    v.z = t[4] | ((unsigned)t[5] << 16);
    v.w = t[6] | ((unsigned)t[7] << 16);
    return v;
}

// x staging: x (length K) goes to LDS zero-padded to nslab whole slabs (uniform trip counts),
// optionally RMS-normalized (rmsnorm with weight nw). Loads are issued in batches of 8 slabs with
// clamped addresses (no divergent branches around them); the first batch is issued by the
// caller before the weight prefetch so that waiting for x does not wait for the weights.
constexpr int kXBatch = 8;

template <bool VEC>
__device__ __forceinline__ void x_load_batch(u32x4 (&v)[kXBatch], const h16 *__restrict__ x, int64_t K, int nslab,
                                             int i0) {
    const int64_t Kp = (K + 7) & ~int64_t(7);
#pragma unroll
    for (int j = 0; j < kXBatch; j++) {
        v[j] = u32x4{0u, 0u, 0u, 0u};
        if (i0 + j < nslab) {  // uniform across the workgroup
            const int64_t k = (int64_t)threadIdx.x * 8 + (int64_t)(i0 + j) * kSlab;
            const bool ok = k < Kp;  // false only in a partial last slab
            v[j] = VEC ? ld16(x + (ok ? k : 0)) : gather8(x, ok ? k : 0, K);
            if (!ok) v[j] = u32x4{0u, 0u, 0u, 0u};
        }
    }
}

template <bool VEC, bool NORM>
__device__ __forceinline__ float x_store_batch(const u32x4 (&v)[kXBatch], h16 *xs, int64_t K, int nslab, int i0,
                                               h16 *xcopy, float ss) {
    const int64_t Kp = (K + 7) & ~int64_t(7);
#pragma unroll
    for (int j = 0; j < kXBatch; j++) {
        if (i0 + j >= nslab) break;
        const int64_t k = (int64_t)threadIdx.x * 8 + (int64_t)(i0 + j) * kSlab;
        st16(xs + k, v[j]);
        if (xcopy && k < Kp) {  // raw (pre-norm) copy of x, written by workgroup 0 only
            if (VEC) {
                st16(xcopy + k, v[j]);
            } else {
                for (int t = 0; t < 8 && k + t < K; t++) xcopy[k + t] = xs[k + t];
            }
        }
        if (NORM) ss = sumsq8(v[j], ss);
    }
    return ss;
}

// Finishes staging after the first batch was loaded into `first`: stores it, loads and stores
// the remaining batches, then applies the RMSNorm scale (each thread to the chunks it loaded, so
// only the sum of squares needs a workgroup exchange).
template <bool VEC, bool NORM>
__device__ __forceinline__ void x_stage_finish(const u32x4 (&first)[kXBatch], h16 *xs, const h16 *__restrict__ x,
                                               int64_t K, int nslab, const h16 *__restrict__ nw, float eps,
                                               float *red, h16 *xcopy) {
    float ss = x_store_batch<VEC, NORM>(first, xs, K, nslab, 0, xcopy, 0.0f);
    for (int i0 = kXBatch; i0 < nslab; i0 += kXBatch) {
        u32x4 v[kXBatch];
        x_load_batch<VEC>(v, x, K, nslab, i0);
        ss = x_store_batch<VEC, NORM>(v, xs, K, nslab, i0, xcopy, ss);
    }
    if (NORM) {
        const int64_t Kp = (K + 7) & ~int64_t(7);
        ss = block_sum<kThreads / kWave>(ss, red);
        const h16 inv = (h16)(1.0f / sqrtf(ss / (float)K + eps));
        for (int i = 0; i < nslab; i++) {
            const int64_t k = (int64_t)threadIdx.x * 8 + (int64_t)i * kSlab;
            if (k >= Kp) break;
            u32x4 w = VEC ? ld16(nw + k) : gather8(nw, k, K);
            st16(xs + k, norm8(ld16(xs + k), w, inv));
        }
    }
}

// x source of one launch: x = xin + m * x_stride, or, with `token` set, row token->token of xin
// (the embedding table: the layer-0 launch of a decode step reads x straight from it and
// workgroup 0 writes the raw row to xcopy, which becomes the residual stream).
struct XSrc {
    const h16 *xin;
    int64_t x_stride;
    const DecodeState *token;
    h16 *xcopy;
};

template <int ROWS, bool VEC, bool NORM, class Epi>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const h16 *__restrict__ W, int64_t N, int64_t K, XSrc src,
                                                        const h16 *__restrict__ nw, float eps, Epi epi) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    h16 *xs = reinterpret_cast<h16 *>(smem_raw);
    __shared__ float red[4 * ROWS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t n0 = (int64_t)blockIdx.x * ROWS;
    const int64_t m = blockIdx.y;
    const int64_t Kp = (K + 7) & ~int64_t(7);
    const int64_t k0 = (int64_t)tid * 8;

    // Rows past N (last group only) re-read row N-1; the epilogue drops them.
    const h16 *wr[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) wr[r] = W + (n0 + r < N ? n0 + r : N - 1) * K;

    // Weights stream through a register double buffer: every ROWS-row slab is requested one
    // slab ahead of its use, so each thread keeps 2 x ROWS 16-byte loads in flight. The slab
    // count is uniform across the workgroup (x is zero-padded in LDS and tail addresses are
    // clamped into the row), so the loop runs under scalar control. The first slab is
    // requested right after x, overlapping its latency with the prologue.
    const int nslab = (int)((Kp + kSlab - 1) / kSlab);
    auto kw = [&](int i) -> int64_t {
        const int64_t k = k0 + (int64_t)i * kSlab;
        return k < Kp ? k : Kp - 8;
    };
    u32x4 wa[ROWS], wb[ROWS];
    auto fetch = [&](u32x4 (&w)[ROWS], int i) {
        const int64_t k = kw(i);
#pragma unroll
        for (int r = 0; r < ROWS; r++) w[r] = VEC ? ld16_stream(wr[r] + k) : gather8(wr[r], k, K);
    };
    float acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) acc[r] = 0.0f;
    auto consume = [&](const u32x4 (&w)[ROWS], int i) {
        const u32x4 xv = ld16(xs + k0 + (int64_t)i * kSlab);  // zero beyond K
#pragma unroll
        for (int r = 0; r < ROWS; r++) acc[r] = dot8(w[r], xv, acc[r]);
    };
    const h16 *x = src.token ? src.xin + src.token->token * src.x_stride : src.xin + m * src.x_stride;
    u32x4 xfirst[kXBatch];
    x_load_batch<VEC>(xfirst, x, K, nslab, 0);
    __builtin_amdgcn_sched_barrier(0);  // keep the x requests ahead of the weight requests
    fetch(wa, 0);
    __builtin_amdgcn_sched_barrier(0);
    const auto pre = epi.template prefetch<ROWS>(n0, m, N, tid);  // epilogue operands, off the tail
    x_stage_finish<VEC, NORM>(xfirst, xs, x, K, nslab, nw, eps, red,
                              (src.xcopy && blockIdx.x == 0) ? src.xcopy : nullptr);
    __syncthreads();

    for (int i = 0; i < nslab; i += 2) {
        if (i + 1 < nslab) fetch(wb, i + 1);
        consume(wa, i);
        if (i + 1 >= nslab) break;
        if (i + 2 < nslab) fetch(wa, i + 2);
        consume(wb, i + 1);
    }

    wave_multi_sum<ROWS>(acc, lane);
    constexpr int G = kWave / ROWS;
    if ((lane & (G - 1)) == 0) red[wave * ROWS + lane / G] = acc[0];
    __syncthreads();
    epi.template apply<ROWS>(n0, m, N, RowSums<ROWS>{red}, tid, pre);
}

// Fixed-shape fast path (K % 8 == 0, 16-byte aligned, NS = ceil(K / 2048) slabs known at
// compile time). Thread t only ever multiplies its own x chunks (k = 8t + 2048i), so x stays in
// registers, RMS-normalized in place; the only workgroup exchange before the dot products is
// the sum of squares (NORM), and plain GEMVs have no barrier at all. Request order: x chunks,
// norm weights, then the first DEPTH weight slabs; weights then stream through a ring of DEPTH
// register buffers, each refilled with the slab DEPTH ahead as soon as it is consumed.

template <int ROWS, int NS, bool NORM, class Epi>
__global__ __launch_bounds__(kThreads) void gemv_fixed_kernel(const h16 *__restrict__ W, int64_t N, int64_t K,
                                                              XSrc src, const h16 *__restrict__ nw, float eps,
                                                              Epi epi) {
    __shared__ float red[4 * ROWS];
    __shared__ float nred[4];  // RMSNorm sum of squares
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t n0 = (int64_t)blockIdx.x * ROWS;
    const int64_t m = blockIdx.y;
    const int k0 = tid * 8, Ki = (int)K;  // K <= NS * 2048 <= 14336
    // 4-row groups address the workgroup's rows as one buffer from row n0 (rows past N read as
    // zeros; their sums are not stored): one 64-bit base per workgroup and 32-bit offsets keep the
    // scalar set-up that every wave runs before its first weight request short (measured on
    // MI355X, µs per launch: QKV 9.58 -> 9.26, O 6.9 -> 6.8, gate/up 34.5 -> 34.2). The 8-row
    // lm_head groups measured 1.5-4 µs slower so, and keep one pointer per row (rows past N re-read
    // row N - 1).
    constexpr bool kBuf = ROWS <= 4;
    const int nrows = N - n0 < ROWS ? (int)(N - n0) : ROWS;
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void *)(W + n0 * K), 0, kBuf ? nrows * Ki * 2 : 0, 0x00020000);
    const h16 *wr[ROWS];
    if constexpr (!kBuf) {
#pragma unroll
        for (int r = 0; r < ROWS; r++) wr[r] = W + (n0 + r < N ? n0 + r : N - 1) * K;
    }
    auto wload = [&](int kc, int r) {  // 16 bytes of row n0 + r at element kc (non-temporal)
        if constexpr (kBuf) return __builtin_amdgcn_raw_buffer_load_b128(rw, kc * 2, r * Ki * 2, 2);
        else return ld16_stream(wr[r] + kc);
    };
    const h16 *x = src.token ? src.xin + src.token->token * src.x_stride : src.xin + m * src.x_stride;

    u32x4 xr[NS], nr[NS];
    bool live[NS];
#pragma unroll
    for (int i = 0; i < NS; i++) {
        const int k = k0 + i * kSlab;
        live[i] = k < Ki;  // false only in a partial last slab
        xr[i] = ld16(x + (live[i] ? k : 0));
        if (NORM) nr[i] = ld16(nw + (live[i] ? k : 0));
    }
    __builtin_amdgcn_sched_barrier(0);
    constexpr int D = NS < kGemvDepth ? NS : kGemvDepth;
    u32x4 wbuf[D][ROWS];
#pragma unroll
    for (int j = 0; j < D; j++) {
        const int k = k0 + j * kSlab;
        const int kc = k < Ki ? k : k0;  // k0 < 2048 <= K; dead lanes of a partial slab re-read slab 0
#pragma unroll
        for (int r = 0; r < ROWS; r++) wbuf[j][r] = wload(kc, r);
    }
    __builtin_amdgcn_sched_barrier(0);
    const auto pre = epi.template prefetch<ROWS>(n0, m, N, tid);  // epilogue operands, off the tail

    float ss = 0.0f;
    h16 *xcopy = (src.xcopy && blockIdx.x == 0) ? src.xcopy : nullptr;
#pragma unroll
    for (int i = 0; i < NS; i++) {
        if (!live[i]) xr[i] = u32x4{0u, 0u, 0u, 0u};
        if (xcopy && live[i]) st16(xcopy + k0 + (int64_t)i * kSlab, xr[i]);
        if (NORM) ss = sumsq8(xr[i], ss);
    }
    if (NORM) {
        ss = block_sum<kThreads / kWave, false>(ss, nred);
        const h16 inv = (h16)(1.0f / sqrtf(ss / (float)K + eps));
#pragma unroll
        for (int i = 0; i < NS; i++) xr[i] = norm8(xr[i], nr[i], inv);  // zero chunks stay zero
    }

    float acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) acc[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < NS; i++) {
#pragma unroll
        for (int r = 0; r < ROWS; r++) acc[r] = dot8(wbuf[i % D][r], xr[i], acc[r]);
        if (i + D < NS) {
            const int k = k0 + (i + D) * kSlab;
            const int kc = k < Ki ? k : k0;  // dead lanes of a partial slab re-read slab 0
#pragma unroll
            for (int r = 0; r < ROWS; r++) wbuf[i % D][r] = wload(kc, r);
        }
    }

    wave_multi_sum<ROWS>(acc, lane);
    constexpr int G = kWave / ROWS;
    if ((lane & (G - 1)) == 0) red[wave * ROWS + lane / G] = acc[0];
    __syncthreads();
    epi.template apply<ROWS>(n0, m, N, RowSums<ROWS>{red}, tid, pre);
}

// Final argmax over ordered partials (one workgroup). Writes *result and/or the decode state:
// next_token, and in autoregressive mode token <- next, pos += 1, step += 1, ring[step] = next.
// Partial g is the first maximum of an index range below partial g + 1's, so the answer is the
// smallest index among the partials holding the largest value, whatever order they are visited
// in: thread t keeps the first maximum of partials t, t + 1024, ... (coalesced loads, 16 in
// flight), then the workgroup takes the largest value and the smallest index holding it (one wave
// reduction and one LDS exchange each, two barriers in all).
constexpr int kFinishThreads = 1024;
constexpr int kFinishWaves = kFinishThreads / kWave;
constexpr int kFinishBatch = 16;
__global__ __launch_bounds__(kFinishThreads) void argmax_finish_kernel(const ArgPart *__restrict__ parts,
                                                                        int64_t count, DecodeState *state,
                                                                        int64_t *ring, int64_t *result) {
    __shared__ float wmax[kFinishWaves];
    __shared__ int32_t widx[kFinishWaves];
    const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    float cv = -INFINITY;
    int32_t ci = INT32_MAX;
    for (int64_t g0 = tid; g0 < count; g0 += (int64_t)kFinishBatch * kFinishThreads) {
        ArgPart v[kFinishBatch];
#pragma unroll
        for (int j = 0; j < kFinishBatch; j++) {
            const int64_t g = g0 + (int64_t)j * kFinishThreads;
            v[j] = g < count ? parts[g] : ArgPart{-INFINITY, -1};
        }
#pragma unroll
        for (int j = 0; j < kFinishBatch; j++)
            if (v[j].v > cv) {  // ascending partials: strict '>' keeps the first maximum
                cv = v[j].v;
                ci = v[j].i;
            }
    }
    const float wm = wave_max(cv);
    if (lane == 0) wmax[wave] = wm;
    __syncthreads();
    float vmax = wmax[0];
#pragma unroll
    for (int w = 1; w < kFinishWaves; w++) vmax = fmaxf(vmax, wmax[w]);
    const int32_t wi = wave_min_i(cv == vmax ? ci : INT32_MAX);
    if (lane == 0) widx[wave] = wi;
    __syncthreads();
    if (tid != 0) return;
    int32_t bi = widx[0];
#pragma unroll
    for (int w = 1; w < kFinishWaves; w++) bi = min(bi, widx[w]);
    const int64_t idx = (vmax > kArgmaxFloor && bi != INT32_MAX && bi >= 0) ? (int64_t)bi : 0;
    if (result) *result = idx;
    if (state) {
        state->next_token = idx;
        if (state->advance) {
            if (ring) ring[state->step % state->ring_cap] = idx;
            state->token = idx;
            state->pos = state->pos + 1;
            state->step = state->step + 1;
        }
    }
}

// ------------------------------------------------------------------ Q8_0 weights
//
// Q8_0 matrices are repacked in HBM as int8 quants [N][K] (rows 32-byte aligned) plus f16 block
// scales [N][K / 32]. Per row and slab a thread makes one 16- or 8-byte quant load and one 2-byte
// scale load, so a wave streams contiguous 1 KiB or 512 B of quants per row.
// Dequantization (dequant_q8x4) reproduces gemm_q8_0 (compute.mojo:1038-1065) exactly:
// w = f16(f16(q) * d); the dot product is v_dot2_f32_f16.
// Rows per group of the Q8_0 decode GEMVs, and row groups per workgroup. Measured on MI355X
// (Llama-3-8B shapes, us per launch): 4 rows beat 8 and 16 on every GEMV; 2 groups per workgroup
// take gate/up from 24.2 to 23.2 but slow the 4096-row GEMVs (QKV 7.7 -> 9.1, O 5.7 -> 6.2), and
// 4 or 8 groups are slower still.
constexpr int kQ8Rows = 4;

// f16 values f16(q_j * d) of 16 quants, as two 8-element chunks.
__device__ __forceinline__ void deq16(u32x4 q, h16 d, u32x4 &o0, u32x4 &o1) {
    unsigned o[8];
    dequant_q8x4(q.x, d, o[0], o[1]);
    dequant_q8x4(q.y, d, o[2], o[3]);
    dequant_q8x4(q.z, d, o[4], o[5]);
    dequant_q8x4(q.w, d, o[6], o[7]);
    o0 = u32x4{o[0], o[1], o[2], o[3]};
    o1 = u32x4{o[4], o[5], o[6], o[7]};
}

// x source of a Q8_0 launch: x itself, or (layer 0) row token->token of the Q8_0 embedding table,
// dequantized in registers, with workgroup 0 writing the row to xcopy (the residual stream).
struct Q8XSrc {
    const h16 *x;
    const int8_t *eq;
    const h16 *ed;
    const DecodeState *token;
    h16 *xcopy;
};

// The Q8_0 twin of gemv_fixed_kernel (K % 32 == 0): thread t multiplies QW quants per row and
// slab (k = QW t + 256 QW i, NS slabs; QW = 16 loads half a block per row, QW = 8 a quarter, so
// K = 2048 or 14336 need no idle lanes). x chunks stay in registers, optionally RMS-normalized
// once per workgroup. A workgroup owns G consecutive groups of ROWS rows; the weight requests run
// D (group, slab) steps ahead of the dot products through a register ring, so the next group's
// rows are in flight during a group's reduction and epilogue, and x is loaded and normalized once
// for G groups.
template <int QW>
struct QVec;  // QW quants of one row
template <>
struct QVec<16> {
    u32x4 v;
    __device__ __forceinline__ static QVec load(const int8_t *p) { return QVec{ld16_stream(p)}; }
    __device__ __forceinline__ static QVec load(__amdgpu_buffer_rsrc_t r, int v, int s) {
        return QVec{__builtin_amdgcn_raw_buffer_load_b128(r, v, s, 2)};
    }
};
template <>
struct QVec<8> {
    u32x2 v;
    __device__ __forceinline__ static QVec load(const int8_t *p) {
        return QVec{__builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p))};
    }
    __device__ __forceinline__ static QVec load(__amdgpu_buffer_rsrc_t r, int v, int s) {
        return QVec{__builtin_amdgcn_raw_buffer_load_b64(r, v, s, 2)};
    }
};
// f16(q * d) of the QW quants as QW / 8 chunks of 8 f16
__device__ __forceinline__ void deq(const QVec<16> &q, h16 d, u32x4 (&o)[2]) { deq16(q.v, d, o[0], o[1]); }
__device__ __forceinline__ void deq(const QVec<8> &q, h16 d, u32x4 (&o)[1]) {
    unsigned w[4];
    dequant_q8x4(q.v.x, d, w[0], w[1]);
    dequant_q8x4(q.v.y, d, w[2], w[3]);
    o[0] = u32x4{w[0], w[1], w[2], w[3]};
}

template <int ROWS, int NS, int G, int QW, bool NORM, class Epi>
__global__ __launch_bounds__(kThreads) void gemv_q8_kernel(const int8_t *__restrict__ Wq, const h16 *__restrict__ Wd,
                                                           int64_t N, int64_t K, Q8XSrc src,
                                                           const h16 *__restrict__ nw, float eps, Epi epi) {
    constexpr int XC = QW / 8;                  // 8-element x chunks per slab
    constexpr int64_t SLAB = (int64_t)kThreads * QW;
    __shared__ float red[G > 1 ? 2 : 1][4 * ROWS];  // alternating per row group: one barrier per group
    __shared__ float nred[4];                      // RMSNorm sum of squares
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t nbase = (int64_t)blockIdx.x * G * ROWS;
    const int64_t k0 = (int64_t)tid * QW;
    const int64_t KB = K / 32;
    // the workgroup's G * ROWS rows through one buffer resource each for quants and scales: 32-bit
    // row offsets in scalar registers, and rows past N read zeros (their sums are never stored)
    const int Ki = (int)K, KBi = (int)KB;
    const int nrows = N - nbase < G * ROWS ? (int)(N - nbase) : G * ROWS;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void *)(Wq + nbase * K), 0, nrows * Ki, 0x00020000);
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc((void *)(Wd + nbase * KB), 0, nrows * KBi * 2, 0x00020000);
    u32x4 xr[NS][XC], nr[NS][XC];
    bool live[NS];
    QVec<QW> eqv[NS];
    h16 edv[NS];
    const bool embed = src.eq != nullptr;
    const int64_t trow = embed ? src.token->token : 0;
#pragma unroll
    for (int i = 0; i < NS; i++) {
        const int64_t k = k0 + (int64_t)i * SLAB;
        live[i] = k < K;  // false in a partial slab (and for every thread beyond K when K < SLAB)
        const int64_t kc = live[i] ? k : 0;
        if (embed) {  // quants and scale of the embedding row; dequantized below
            eqv[i] = QVec<QW>::load(src.eq + trow * K + kc);
            edv[i] = src.ed[trow * KB + kc / 32];
        } else {
#pragma unroll
            for (int c = 0; c < XC; c++) xr[i][c] = ld16(src.x + kc + 8 * c);
        }
        if (NORM) {
#pragma unroll
            for (int c = 0; c < XC; c++) nr[i][c] = ld16(nw + kc + 8 * c);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    const int64_t kf = k0 < K ? k0 : 0;
    // step st = (group st / NS, slab st % NS); D steps in flight through a register ring
    constexpr int T = G * NS, D = T < kGemvDepth ? T : kGemvDepth;
    QVec<QW> qb[D][ROWS];
    h16 db[D][ROWS];
    auto request = [&](int st) {
        const int g = st / NS, i = st % NS;
        const int64_t k = k0 + (int64_t)i * SLAB;
        const int kc = (int)(k < K ? k : kf);  // dead lanes of a partial slab re-read their first chunk
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            const int rr = g * ROWS + r;
            qb[st % D][r] = QVec<QW>::load(rq, kc, rr * Ki);
            db[st % D][r] = __builtin_bit_cast(h16, __builtin_amdgcn_raw_buffer_load_b16(rd, (kc >> 5) * 2, rr * KBi * 2, 0));
        }
    };
#pragma unroll
    for (int st = 0; st < D; st++) request(st);
    __builtin_amdgcn_sched_barrier(0);
    using Pre = decltype(epi.template prefetch<ROWS>(0, 0, N, tid));
    Pre pre[G];
#pragma unroll
    for (int g = 0; g < G; g++)
        if (g * NS < D) pre[g] = epi.template prefetch<ROWS>(nbase + (int64_t)g * ROWS, 0, N, tid);

    float ss = 0.0f;
    h16 *xcopy = (src.xcopy && blockIdx.x == 0) ? src.xcopy : nullptr;
#pragma unroll
    for (int i = 0; i < NS; i++) {
        if (embed) deq(eqv[i], edv[i], xr[i]);
#pragma unroll
        for (int c = 0; c < XC; c++) {
            if (!live[i]) xr[i][c] = u32x4{0u, 0u, 0u, 0u};
            if (xcopy && live[i]) st16(xcopy + k0 + (int64_t)i * SLAB + 8 * c, xr[i][c]);
            if (NORM) ss = sumsq8(xr[i][c], ss);
        }
    }
    if (NORM) {
        ss = block_sum<kThreads / kWave, false>(ss, nred);
        const h16 inv = (h16)(1.0f / sqrtf(ss / (float)K + eps));
#pragma unroll
        for (int i = 0; i < NS; i++)
#pragma unroll
            for (int c = 0; c < XC; c++) xr[i][c] = norm8(xr[i][c], nr[i][c], inv);
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
        float acc[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; r++) acc[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const int st = g * NS + i;
#pragma unroll
            for (int r = 0; r < ROWS; r++) {
                u32x4 w[XC];
                deq(qb[st % D][r], db[st % D][r], w);
#pragma unroll
                for (int c = 0; c < XC; c++) acc[r] = dot8(w[c], xr[i][c], acc[r]);
            }
            if (st + D < T) {
                request(st + D);
                const int gn = (st + D) / NS;
                if ((st + D) % NS == 0) pre[gn] = epi.template prefetch<ROWS>(nbase + (int64_t)gn * ROWS, 0, N, tid);
            }
        }
        wave_multi_sum<ROWS>(acc, lane);
        constexpr int GW = kWave / ROWS;
        float *rg = red[g & (G > 1 ? 1 : 0)];  // group g + 2 rewrites it only after group g + 1's barrier
        if ((lane & (GW - 1)) == 0) rg[wave * ROWS + lane / GW] = acc[0];
        __syncthreads();
        epi.template apply<ROWS>(nbase + (int64_t)g * ROWS, 0, N, RowSums<ROWS>{rg}, tid, pre[g]);
    }
}

template <int ROWS, int G, bool NORM, class Epi>
static int32_t gemv_q8_dispatch(hipStream_t s, const void *Wq, const void *Wd, int64_t N, int64_t K, const Q8XSrc &src,
                                const void *nw, float eps, const Epi &epi, const char *name) {
    const void *xp = src.eq ? (const void *)src.eq : (const void *)src.x;
    if (K % 32 != 0 || ((uintptr_t)Wq & 15) || ((uintptr_t)xp & 15) || (NORM && ((uintptr_t)nw & 15)) ||
        (src.xcopy && ((uintptr_t)src.xcopy & 15)))
        return fail(AESIR_ERR_UNSUPPORTED, "%s: Q8_0 GEMV needs K %% 32 == 0 and 16-byte aligned rows", name);
    const dim3 grid((unsigned)((N + ROWS * G - 1) / (ROWS * G)));
    if (grid.x == 0) return AESIR_OK;
    // 8 quants per thread below K = 4096 (a 4096-wide slab would leave half the lanes idle at K =
    // 2048), else 16. Measured on MI355X: TinyLlama Q8_0 decode 1316 -> 1399 tok/s with 8; at
    // K = 14336 8-quant slabs (7 whole ones) lose to 16-quant ones (3.5): 17.4 against 14.2 us.
    const bool qw8 = K < 4096;
    const int64_t ns = qw8 ? (K + 2047) / 2048 : (K + 4095) / 4096;
#define AESIR_GEMV_Q8(QWV, NSV)                                                                            \
    case NSV:                                                                                             \
        hipLaunchKernelGGL((gemv_q8_kernel<ROWS, NSV, G, QWV, NORM, Epi>), grid, dim3(kThreads), 0, s,    \
                           (const int8_t *)Wq, (const h16 *)Wd, N, K, src, (const h16 *)nw, eps, epi);    \
        break;
    if (qw8) {
        switch (ns) {
            AESIR_GEMV_Q8(8, 1)
            AESIR_GEMV_Q8(8, 2)
            AESIR_GEMV_Q8(8, 3)
            AESIR_GEMV_Q8(8, 4)
            AESIR_GEMV_Q8(8, 5)
            AESIR_GEMV_Q8(8, 6)
            AESIR_GEMV_Q8(8, 7)
            AESIR_GEMV_Q8(8, 8)
            default:
                return fail(AESIR_ERR_UNSUPPORTED, "%s: Q8_0 GEMV with K = %lld exceeds 28672", name, (long long)K);
        }
    } else {
        switch (ns) {
            AESIR_GEMV_Q8(16, 1)
            AESIR_GEMV_Q8(16, 2)
            AESIR_GEMV_Q8(16, 3)
            AESIR_GEMV_Q8(16, 4)
            AESIR_GEMV_Q8(16, 5)
            AESIR_GEMV_Q8(16, 6)
            AESIR_GEMV_Q8(16, 7)
            default:
                return fail(AESIR_ERR_UNSUPPORTED, "%s: Q8_0 GEMV with K = %lld exceeds 28672", name, (long long)K);
        }
    }
#undef AESIR_GEMV_Q8
    AESIR_LAUNCH_CHECK(name);
    return AESIR_OK;
}

// ------------------------------------------------------------------ launchers

static int64_t lds_bytes(int64_t K) { return (((K + 7) & ~int64_t(7)) + kSlab - 1) / kSlab * kSlab * 2; }

template <class KernelPtr>
static int32_t ensure_lds(KernelPtr k, int64_t bytes) {
    if (bytes > 160 * 1024) return fail(AESIR_ERR_UNSUPPORTED, "gemv: K=%lld exceeds the LDS staging limit", (long long)(bytes / 2));
    if (bytes > 64 * 1024)
        AESIR_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    return AESIR_OK;
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

template <int ROWS, bool NORM, class Epi>
static int32_t gemv_dispatch(hipStream_t s, const void *W, int64_t N, int64_t K, const XSrc &src, int64_t M,
                             const void *nw, float eps, const Epi &epi, const char *name) {
    const bool vec = (K % 8 == 0) && aligned16(W) && aligned16(src.xin) && (src.x_stride % 8 == 0) &&
                     (!NORM || aligned16(nw)) && (!src.xcopy || aligned16(src.xcopy));
    const int64_t lds = lds_bytes(K);
    const dim3 grid((unsigned)((N + ROWS - 1) / ROWS), (unsigned)M);
    if (grid.x == 0 || grid.y == 0) return AESIR_OK;
    const int64_t ns = (K + kSlab - 1) / kSlab;
    if (vec && ns <= 8 && K >= kSlab) {
        switch (ns) {
#define AESIR_GEMV_FIXED(NSV)                                                                                    \
    case NSV:                                                                                                   \
        hipLaunchKernelGGL((gemv_fixed_kernel<ROWS, NSV, NORM, Epi>), grid, dim3(kThreads), 0, s, (const h16 *)W, N, K, \
                           src, (const h16 *)nw, eps, epi);                                                      \
        break;
            AESIR_GEMV_FIXED(1)
            AESIR_GEMV_FIXED(2)
            AESIR_GEMV_FIXED(3)
            AESIR_GEMV_FIXED(4)
            AESIR_GEMV_FIXED(5)
            AESIR_GEMV_FIXED(6)
            AESIR_GEMV_FIXED(7)
            AESIR_GEMV_FIXED(8)
#undef AESIR_GEMV_FIXED
        }
        AESIR_LAUNCH_CHECK(name);
        return AESIR_OK;
    }
    if (vec) {
        auto k = gemv_kernel<ROWS, true, NORM, Epi>;
        AESIR_TRY(ensure_lds(k, lds));
        hipLaunchKernelGGL(k, grid, dim3(kThreads), (unsigned)lds, s, (const h16 *)W, N, K, src, (const h16 *)nw, eps,
                           epi);
    } else {
        auto k = gemv_kernel<ROWS, false, NORM, Epi>;
        AESIR_TRY(ensure_lds(k, lds));
        hipLaunchKernelGGL(k, grid, dim3(kThreads), (unsigned)lds, s, (const h16 *)W, N, K, src, (const h16 *)nw, eps,
                           epi);
    }
    AESIR_LAUNCH_CHECK(name);
    return AESIR_OK;
}

// Rows per workgroup of the decode-step GEMVs. 4 rows (twice the workgroups of 8) shortens the
// ramp and the tail of a launch; measured on MI355X: 4096 x 4096 8.2 -> 7.4 us, 6144 x 4096
// 10.7 -> 9.7 us, 4096 x 14336 20.3 -> 19.8 us, gate/up 28672 x 4096 37.1 -> 35.0 us.
constexpr int kRowsSmall = 4;

int32_t launch_gemm_f16(aesir_ctx *ctx, const void *A, int64_t M, int64_t K, const void *B, int64_t N, void *C) {
    if (M > 65535) return fail(AESIR_ERR_UNSUPPORTED, "gemm_f16: more than 65535 rows of A");
    EpiStore e{(h16 *)C, N};
    return gemv_dispatch<kRowsSmall, false>(ctx->stream, B, N, K, XSrc{(const h16 *)A, K, nullptr, nullptr}, M, nullptr,
                                            0.0f, e, "gemv_store");
}

int32_t launch_qkv_rope_kv(hipStream_t s, const QkvArgs &a) {
    EpiQkv e{(h16 *)a.q_out, (h16 *)a.k_cache, (h16 *)a.v_cache, (const h16x2 *)a.rope, a.state,
             a.dim, a.kvd, a.head_dim, a.max_seq};
    if (qf_type(a.wq.type)) return launch_qf_qkv_rope_kv(s, a, e);
    if (a.w_scale) {  // Q8_0 weights (and, for layer 0, a Q8_0 embedding table)
        const Q8XSrc src = a.embd ? Q8XSrc{nullptr, (const int8_t *)a.embd, (const h16 *)a.embd_scale, a.state, (h16 *)a.x}
                                  : Q8XSrc{(const h16 *)a.x, nullptr, nullptr, nullptr, nullptr};
        return gemv_q8_dispatch<kQ8Rows, 1, true>(s, a.w, a.w_scale, a.dim + 2 * a.kvd, a.dim, src, a.norm_w, a.eps, e,
                                                  "gemv_q8_qkv_rope_kv");
    }
    XSrc src = a.embd ? XSrc{(const h16 *)a.embd, a.dim, a.state, (h16 *)a.x} : XSrc{(const h16 *)a.x, 0, nullptr, nullptr};
    return gemv_dispatch<kRowsSmall, true>(s, a.w, a.dim + 2 * a.kvd, a.dim, src, 1, a.norm_w, a.eps, e, "gemv_qkv_rope_kv");
}

int32_t launch_gemv_residual(hipStream_t s, const void *w, int64_t N, int64_t K, const void *x_in, void *x,
                             const void *w_scale) {
    EpiResidual e{(h16 *)x};
    if (w_scale)
        return gemv_q8_dispatch<kQ8Rows, 1, false>(s, w, w_scale, N, K, Q8XSrc{(const h16 *)x_in, nullptr, nullptr, nullptr, nullptr},
                                                   nullptr, 0.0f, e, "gemv_q8_residual");
    return gemv_dispatch<kRowsSmall, false>(s, w, N, K, XSrc{(const h16 *)x_in, 0, nullptr, nullptr}, 1, nullptr, 0.0f, e,
                                            "gemv_residual");
}

int32_t launch_gate_up_swiglu(hipStream_t s, const void *x, const void *norm_w, float eps, const void *w,
                              int64_t ffn, int64_t dim, void *act, const void *w_scale) {
    EpiSwiglu e{(h16 *)act};
    if (w_scale)
        return gemv_q8_dispatch<kQ8Rows, 2, true>(s, w, w_scale, 2 * ffn, dim, Q8XSrc{(const h16 *)x, nullptr, nullptr, nullptr, nullptr},
                                                  norm_w, eps, e, "gemv_q8_gate_up");
    return gemv_dispatch<kRowsSmall, true>(s, w, 2 * ffn, dim, XSrc{(const h16 *)x, 0, nullptr, nullptr}, 1, norm_w,
                                           eps, e, "gemv_gate_up_swiglu");
}

int64_t lm_head_groups(int64_t vocab) { return (vocab + 7) / 8; }

int32_t launch_lm_head(hipStream_t s, const LmHeadArgs &a) {
    EpiLmHead e{(h16 *)a.logits, (ArgPart *)a.partials};
    if (qf_type(a.wq.type)) return launch_qf_lm_head(s, a, e);
    if (a.w_scale)
        return gemv_q8_dispatch<8, 1, true>(s, a.w, a.w_scale, a.vocab, a.dim, Q8XSrc{(const h16 *)a.x, nullptr, nullptr, nullptr, nullptr},
                                         a.norm_w, a.eps, e, "gemv_q8_lm_head");
    return gemv_dispatch<8, true>(s, a.w, a.vocab, a.dim, XSrc{(const h16 *)a.x, 0, nullptr, nullptr}, 1, a.norm_w,
                                  a.eps, e, "gemv_lm_head");
}

int32_t launch_argmax_finish(hipStream_t s, const void *partials, int64_t count, DecodeState *state, int64_t *ring,
                             int64_t *result) {
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(kFinishThreads), 0, s, (const ArgPart *)partials, count,
                       state, ring, result);
    AESIR_LAUNCH_CHECK("argmax_finish_kernel");
    return AESIR_OK;
}

int32_t launch_lm_head_argmax(hipStream_t s, const LmHeadArgs &a) {
    AESIR_TRY(launch_lm_head(s, a));
    return launch_argmax_finish(s, a.partials, lm_head_groups(a.vocab), a.state, a.ring, nullptr);
}

// ------------------------------------------------------------------ standalone argmax

// Stage 1 of the standalone argmax: each workgroup scans a contiguous chunk in ascending order
// (strict '>') and writes one ordered partial; argmax_finish_kernel reduces them.
__global__ __launch_bounds__(kThreads) void argmax_kernel(const h16 *__restrict__ x, int64_t n, int64_t chunk,
                                                          ArgPart *parts) {
    __shared__ ArgPart tree[kThreads];
    const int tid = threadIdx.x;
    const int64_t base = (int64_t)blockIdx.x * chunk;
    const int64_t end = base + chunk < n ? base + chunk : n;
    const int64_t per = (chunk + kThreads - 1) / kThreads;
    ArgPart cur{-INFINITY, -1};
    float cv = kArgmaxFloor;
    for (int64_t i = base + (int64_t)tid * per; i < base + (int64_t)(tid + 1) * per && i < end; i++) {
        float v = (float)x[i];
        if (v > cv) {
            cv = v;
            cur = ArgPart{v, (int32_t)i};
        }
    }
    tree[tid] = cur;
    __syncthreads();
    for (int st = 1; st < kThreads; st <<= 1) {
        ArgPart a = tree[tid];
        if ((tid & (2 * st - 1)) == 0 && tid + st < kThreads) a = arg_combine(a, tree[tid + st]);
        __syncthreads();
        tree[tid] = a;
        __syncthreads();
    }
    if (tid == 0) parts[blockIdx.x] = tree[0];
}

int32_t launch_argmax(hipStream_t s, const void *logits, int64_t n, void *partials, int64_t max_parts, int64_t *result) {
    int64_t chunk = 2048;  // 8 elements per thread per workgroup
    int64_t groups = (n + chunk - 1) / chunk;
    if (groups > max_parts) {
        groups = max_parts;
        chunk = (n + groups - 1) / groups;
    }
    hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)groups), dim3(kThreads), 0, s, (const h16 *)logits, n, chunk,
                       (ArgPart *)partials);
    AESIR_LAUNCH_CHECK("argmax_kernel");
    return launch_argmax_finish(s, partials, groups, nullptr, nullptr, result);
}

}  // namespace aesir
