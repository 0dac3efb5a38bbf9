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
#include "kernels.hpp"

namespace aesir {

constexpr int kThreads = 256;
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

// Stages x (length K, zero-padded to a multiple of 8) into LDS; with NORM, applies rmsnorm with
// weight nw. Each thread normalizes exactly the chunks it loaded, so only the sum of squares
// needs a workgroup exchange.
template <bool VEC, bool NORM>
__device__ __forceinline__ void stage_x(h16 *xs, const h16 *__restrict__ x, int64_t K, const h16 *__restrict__ nw,
                                        float eps, float *red) {
    const int tid = threadIdx.x;
    const int64_t Kp = (K + 7) & ~int64_t(7);
    float ss = 0.0f;
    for (int64_t k = (int64_t)tid * 8; k < Kp; k += kSlab) {
        u32x4 v = VEC ? ld16(x + k) : gather8(x, k, K);
        st16(xs + k, v);
        if (NORM) ss = sumsq8(v, ss);
    }
    if (NORM) {
        ss = block_sum<kThreads / kWave>(ss, red);
        const h16 inv = (h16)(1.0f / sqrtf(ss / (float)K + eps));
        for (int64_t k = (int64_t)tid * 8; k < Kp; k += kSlab) {
            u32x4 w = VEC ? ld16(nw + k) : gather8(nw, k, K);
            st16(xs + k, norm8(ld16(xs + k), w, inv));
        }
    }
}

template <int ROWS, bool VEC, bool NORM, class Epi>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const h16 *__restrict__ W, int64_t N, int64_t K,
                                                        const h16 *__restrict__ xin, int64_t x_stride,
                                                        const h16 *__restrict__ nw, float eps, Epi epi) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    h16 *xs = reinterpret_cast<h16 *>(smem_raw);
    __shared__ float red[4 * ROWS];
    __shared__ float sums[ROWS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t n0 = (int64_t)blockIdx.x * ROWS;
    const int64_t m = blockIdx.y;

    stage_x<VEC, NORM>(xs, xin + m * x_stride, K, nw, eps, red);
    __syncthreads();

    // Rows past N (last group only) re-read row N-1; the epilogue drops them.
    const h16 *wr[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) wr[r] = W + (n0 + r < N ? n0 + r : N - 1) * K;

    float acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) acc[r] = 0.0f;
    const int64_t Kp = (K + 7) & ~int64_t(7);
#pragma unroll 2
    for (int64_t k = (int64_t)tid * 8; k < Kp; k += kSlab) {
        const u32x4 xv = ld16(xs + k);
        u32x4 wv[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; r++) wv[r] = VEC ? ld16_stream(wr[r] + k) : gather8(wr[r], k, K);
#pragma unroll
        for (int r = 0; r < ROWS; r++) acc[r] = dot8(wv[r], xv, acc[r]);
    }

    wave_multi_sum<ROWS>(acc, lane);
    constexpr int G = kWave / ROWS;
    if ((lane & (G - 1)) == 0) red[wave * ROWS + lane / G] = acc[0];
    __syncthreads();
    if (tid < ROWS) sums[tid] = (red[tid] + red[ROWS + tid]) + (red[2 * ROWS + tid] + red[3 * ROWS + tid]);
    __syncthreads();
    epi.template apply<ROWS>(n0, m, N, sums, tid);
}

// ------------------------------------------------------------------ epilogues

struct EpiStore {
    h16 *y;
    int64_t ldy;
    template <int ROWS>
    __device__ __forceinline__ void apply(int64_t n0, int64_t m, int64_t N, const float *s, int tid) const {
        if (tid < ROWS && n0 + tid < N) y[m * ldy + n0 + tid] = (h16)s[tid];
    }
};

// O projection / down projection: x = f16(f16(acc) + x)  (inference.mojo:227-232, 268-273).
struct EpiResidual {
    h16 *x;
    template <int ROWS>
    __device__ __forceinline__ void apply(int64_t n0, int64_t, int64_t N, const float *s, int tid) const {
        if (tid < ROWS && n0 + tid < N) x[n0 + tid] = hadd((h16)s[tid], x[n0 + tid]);
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
    template <int ROWS>
    __device__ __forceinline__ void apply(int64_t n0, int64_t, int64_t N, const float *s, int tid) const {
        static_assert(ROWS % 2 == 0, "pairs must stay in one workgroup");
        if (tid >= ROWS / 2) return;
        const int64_t n = n0 + 2 * tid;
        if (n >= N) return;
        const h16 s0 = (h16)s[2 * tid], s1 = (h16)s[2 * tid + 1];
        const int64_t pos = state->pos;
        const int64_t slot = pos % max_seq;
        if (n < dim + kvd) {
            const int64_t nn = n < dim ? n : n - dim;
            const h16x2 cs = rope[pos * (hd / 2) + ((nn % hd) >> 1)];
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
    __device__ __forceinline__ void apply(int64_t n0, int64_t, int64_t N, const float *s, int tid) const {
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

// Final argmax over `count` ordered partials by one workgroup (256 threads); returns the
// reference's answer (0 if nothing exceeds the floor) to every thread.
__device__ int64_t argmax_finish(const ArgPart *parts, int64_t count) {
    __shared__ ArgPart tree[kThreads];
    const int tid = threadIdx.x;
    const int64_t per = (count + kThreads - 1) / kThreads;
    ArgPart cur{-INFINITY, -1};
    for (int64_t g = (int64_t)tid * per; g < (int64_t)(tid + 1) * per && g < count; g++) {
        ArgPart p = parts[g];
        cur = arg_combine(cur, p);
    }
    tree[tid] = cur;
    __syncthreads();
    for (int s = 1; s < kThreads; s <<= 1) {
        ArgPart a = tree[tid];
        if ((tid & (2 * s - 1)) == 0 && tid + s < kThreads) a = arg_combine(a, tree[tid + s]);
        __syncthreads();
        tree[tid] = a;
        __syncthreads();
    }
    ArgPart best = tree[0];
    __syncthreads();
    return (best.v > kArgmaxFloor && best.i >= 0) ? (int64_t)best.i : 0;
}

// Per-group scan of the ROWS logits of one workgroup in ascending order.
template <int ROWS>
__device__ __forceinline__ ArgPart group_scan(int64_t n0, int64_t N, const float *s) {
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

struct EpiLmHead {
    h16 *logits;
    ArgPart *parts;
    uint32_t *counter;
    DecodeState *state;
    int64_t *ring;
    template <int ROWS>
    __device__ __forceinline__ void apply(int64_t n0, int64_t, int64_t N, const float *s, int tid) const {
        __shared__ int s_last;
        if (tid < ROWS && n0 + tid < N) logits[n0 + tid] = (h16)s[tid];
        if (tid == 0) {
            parts[blockIdx.x] = group_scan<ROWS>(n0, N, s);
            s_last = arrive_is_last(counter, gridDim.x) ? 1 : 0;
        }
        __syncthreads();
        if (!s_last) return;
        last_block_acquire();
        const int64_t idx = argmax_finish(parts, gridDim.x);
        if (tid == 0) {
            state->next_token = idx;
            if (state->advance) {
                if (ring) ring[state->step % state->ring_cap] = idx;
                state->token = idx;
                state->pos = state->pos + 1;
                state->step = state->step + 1;
            }
            *counter = 0;
        }
    }
};

// ------------------------------------------------------------------ launchers

static int64_t lds_bytes(int64_t K) { return ((K + 7) & ~int64_t(7)) * 2; }

template <class KernelPtr>
static int32_t ensure_lds(KernelPtr k, int64_t bytes) {
    if (bytes > 160 * 1024) return fail(AESIR_ERR_UNSUPPORTED, "gemv: K=%lld exceeds the LDS staging limit", (long long)(bytes / 2));
    if (bytes > 64 * 1024)
        AESIR_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    return AESIR_OK;
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

template <int ROWS, bool NORM, class Epi>
static int32_t gemv_dispatch(hipStream_t s, const void *W, int64_t N, int64_t K, const void *x, int64_t x_stride,
                             int64_t M, const void *nw, float eps, const Epi &epi, const char *name) {
    const bool vec = (K % 8 == 0) && aligned16(W) && aligned16(x) && (x_stride % 8 == 0) && (!NORM || aligned16(nw));
    const int64_t lds = lds_bytes(K);
    const dim3 grid((unsigned)((N + ROWS - 1) / ROWS), (unsigned)M);
    if (grid.x == 0 || grid.y == 0) return AESIR_OK;
    if (vec) {
        auto k = gemv_kernel<ROWS, true, NORM, Epi>;
        AESIR_TRY(ensure_lds(k, lds));
        hipLaunchKernelGGL(k, grid, dim3(kThreads), (unsigned)lds, s, (const h16 *)W, N, K, (const h16 *)x, x_stride,
                           (const h16 *)nw, eps, epi);
    } else {
        auto k = gemv_kernel<ROWS, false, NORM, Epi>;
        AESIR_TRY(ensure_lds(k, lds));
        hipLaunchKernelGGL(k, grid, dim3(kThreads), (unsigned)lds, s, (const h16 *)W, N, K, (const h16 *)x, x_stride,
                           (const h16 *)nw, eps, epi);
    }
    AESIR_LAUNCH_CHECK(name);
    return AESIR_OK;
}

int32_t launch_gemm_f16(aesir_ctx *ctx, const void *A, int64_t M, int64_t K, const void *B, int64_t N, void *C) {
    if (M > 65535) return fail(AESIR_ERR_UNSUPPORTED, "gemm_f16: more than 65535 rows of A");
    EpiStore e{(h16 *)C, N};
    return gemv_dispatch<8, false>(ctx->stream, B, N, K, A, K, M, nullptr, 0.0f, e, "gemv_store");
}

int32_t launch_qkv_rope_kv(hipStream_t s, const QkvArgs &a) {
    EpiQkv e{(h16 *)a.q_out, (h16 *)a.k_cache, (h16 *)a.v_cache, (const h16x2 *)a.rope, a.state,
             a.dim, a.kvd, a.head_dim, a.max_seq};
    return gemv_dispatch<8, true>(s, a.w, a.dim + 2 * a.kvd, a.dim, a.x, 0, 1, a.norm_w, a.eps, e, "gemv_qkv_rope_kv");
}

int32_t launch_gemv_residual(hipStream_t s, const void *w, int64_t N, int64_t K, const void *x_in, void *x) {
    EpiResidual e{(h16 *)x};
    return gemv_dispatch<8, false>(s, w, N, K, x_in, 0, 1, nullptr, 0.0f, e, "gemv_residual");
}

int32_t launch_gate_up_swiglu(hipStream_t s, const void *x, const void *norm_w, float eps, const void *w,
                              int64_t ffn, int64_t dim, void *act) {
    EpiSwiglu e{(h16 *)act};
    return gemv_dispatch<8, true>(s, w, 2 * ffn, dim, x, 0, 1, norm_w, eps, e, "gemv_gate_up_swiglu");
}

int64_t lm_head_groups(int64_t vocab) { return (vocab + 7) / 8; }

int32_t launch_lm_head_argmax(hipStream_t s, const LmHeadArgs &a) {
    EpiLmHead e{(h16 *)a.logits, (ArgPart *)a.partials, a.counter, a.state, a.ring};
    return gemv_dispatch<8, true>(s, a.w, a.vocab, a.dim, a.x, 0, 1, a.norm_w, a.eps, e, "gemv_lm_head_argmax");
}

// ------------------------------------------------------------------ standalone argmax

// Stage 1: each workgroup scans a contiguous chunk in ascending order (strict '>').
__global__ __launch_bounds__(kThreads) void argmax_kernel(const h16 *__restrict__ x, int64_t n, int64_t chunk,
                                                          ArgPart *parts, uint32_t *counter, int64_t *result) {
    __shared__ ArgPart tree[kThreads];
    __shared__ int s_last;
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
    for (int s = 1; s < kThreads; s <<= 1) {
        ArgPart a = tree[tid];
        if ((tid & (2 * s - 1)) == 0 && tid + s < kThreads) a = arg_combine(a, tree[tid + s]);
        __syncthreads();
        tree[tid] = a;
        __syncthreads();
    }
    if (tid == 0) {
        parts[blockIdx.x] = tree[0];
        s_last = arrive_is_last(counter, gridDim.x) ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    last_block_acquire();
    const int64_t idx = argmax_finish(parts, gridDim.x);
    if (tid == 0) {
        *result = idx;
        *counter = 0;
    }
}

int32_t launch_argmax(hipStream_t s, const void *logits, int64_t n, void *partials, int64_t max_parts,
                      uint32_t *counter, int64_t *result) {
    // 8 elements per thread per group keeps ~2K groups at n = 128256 ... 16 groups minimum work
    int64_t chunk = 2048;
    int64_t groups = (n + chunk - 1) / chunk;
    if (groups > max_parts) {
        groups = max_parts;
        chunk = (n + groups - 1) / groups;
    }
    hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)groups), dim3(kThreads), 0, s, (const h16 *)logits, n, chunk,
                       (ArgPart *)partials, counter, result);
    AESIR_LAUNCH_CHECK("argmax_kernel");
    return AESIR_OK;
}

}  // namespace aesir
