// Elementwise and row-reduction kernels of the decode path for gfx950: standalone RMSNorm, RoPE,
// SiLU, SwiGLU, residual add, embedding copy, KV append, and the seeded device-side init.
// All are HBM/latency bound; every f16 rounding point of the reference is kept (see device.hpp).
#include "device.hpp"
#include "kernels.hpp"

namespace aesir {

constexpr int kEThreads = 256;

static unsigned grid_for(int64_t n, int64_t per_block) {
    int64_t g = (n + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > 1048576) g = 1048576;
    return (unsigned)g;
}

// ------------------------------------------------------------------ rmsnorm
// One workgroup per row (compute.mojo:2178-2204): f32 sum of squares, inv = f16(1/sqrt(ss/N+eps)),
// x = f16(f16(x * inv) * w).
__global__ __launch_bounds__(kEThreads) void rmsnorm_kernel(h16 *__restrict__ T, int64_t cols,
                                                            const h16 *__restrict__ w, float eps) {
    __shared__ float red[kEThreads / kWave];
    h16 *x = T + (int64_t)blockIdx.x * cols;
    float ss = 0.0f;
    for (int64_t c = threadIdx.x; c < cols; c += kEThreads) {
        float v = (float)x[c];
        ss = fmaf(v, v, ss);
    }
    ss = block_sum<kEThreads / kWave>(ss, red);
    const h16 inv = (h16)(1.0f / sqrtf(ss / (float)cols + eps));
    for (int64_t c = threadIdx.x; c < cols; c += kEThreads) x[c] = hmul(hmul(x[c], inv), w[c]);
}

int32_t launch_rmsnorm(hipStream_t s, void *T, int64_t rows, int64_t cols, const void *w, float eps) {
    if (rows > 2147483647) return fail(AESIR_ERR_UNSUPPORTED, "rmsnorm: too many rows");
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(kEThreads), 0, s, (h16 *)T, cols, (const h16 *)w, eps);
    AESIR_LAUNCH_CHECK("rmsnorm_kernel");
    return AESIR_OK;
}

// ------------------------------------------------------------------ rope
// One thread per (row, pair index j, head): the reference's f16 rotation (compute.mojo:2232-2244)
// with cos/sin from the host-built table at position start_pos + row.
__global__ __launch_bounds__(kEThreads) void rope_kernel(h16 *__restrict__ Q, int64_t q_rows, int64_t q_cols,
                                                         h16 *__restrict__ K, int64_t k_cols, int64_t start_pos,
                                                         int64_t hd, const h16x2 *__restrict__ table) {
    const int64_t half = hd / 2;
    const int64_t pairs_q = q_cols / 2, pairs_k = k_cols / 2;
    const int64_t per_row = pairs_q + pairs_k;
    const int64_t total = q_rows * per_row;
    for (int64_t i = (int64_t)blockIdx.x * kEThreads + threadIdx.x; i < total; i += (int64_t)gridDim.x * kEThreads) {
        const int64_t r = i / per_row, e = i % per_row;
        h16 *p = e < pairs_q ? Q + r * q_cols + 2 * e : K + r * k_cols + 2 * (e - pairs_q);
        const int64_t col = e < pairs_q ? 2 * e : 2 * (e - pairs_q);
        const h16x2 cs = table[(start_pos + r) * half + ((col % hd) >> 1)];
        const h16 a = p[0], b = p[1];
        p[0] = hsub(hmul(a, cs.x), hmul(b, cs.y));
        p[1] = hadd(hmul(a, cs.y), hmul(b, cs.x));
    }
}

// Vector form for head_dim % 8 == 0 and 16-byte aligned rows: one thread per 8 elements (4 pairs,
// one 16-byte load and store) and the pairs' 4 (cos, sin) entries in one 16-byte table load; grid
// (column chunks, row). Same per-pair f16 arithmetic as rope_kernel.
__global__ __launch_bounds__(kEThreads) void rope_vec_kernel(h16 *__restrict__ Q, int64_t q_cols, h16 *__restrict__ K,
                                                             int64_t k_cols, int64_t start_pos, int64_t hd,
                                                             const h16x2 *__restrict__ table) {
    const int64_t r = blockIdx.y;
    const int cq = (int)(q_cols / 8), ck = (int)(k_cols / 8);
    const h16x2 *trow = table + (start_pos + r) * (hd / 2);
    for (int c = blockIdx.x * kEThreads + threadIdx.x; c < cq + ck; c += gridDim.x * kEThreads) {
        h16 *p = c < cq ? Q + r * q_cols + 8 * (int64_t)c : K + r * k_cols + 8 * (int64_t)(c - cq);
        const int col = c < cq ? 8 * c : 8 * (c - cq);
        const u32x4 v = ld16(p);
        const u32x4 t = ld16(trow + ((col % hd) >> 1));
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const h16x2 ab = as_h2(v[j]), cs = as_h2(t[j]);
            const h16x2 rot = {hsub(hmul(ab.x, cs.x), hmul(ab.y, cs.y)), hadd(hmul(ab.x, cs.y), hmul(ab.y, cs.x))};
            o[j] = h2_bits(rot);
        }
        st16(p, o);
    }
}

int32_t launch_rope(hipStream_t s, void *Q, int64_t q_rows, int64_t q_cols, void *K, int64_t k_cols,
                    int64_t start_pos, int64_t head_dim, const void *table) {
    if (head_dim % 8 == 0 && q_cols % 8 == 0 && k_cols % 8 == 0 && q_rows <= 65535 && q_cols + k_cols < (1LL << 31) &&
        (((uintptr_t)Q | (uintptr_t)K | (uintptr_t)table) & 15) == 0) {
        const int64_t chunks = (q_cols + k_cols) / 8;
        hipLaunchKernelGGL(rope_vec_kernel, dim3(grid_for(chunks, kEThreads), (unsigned)q_rows), dim3(kEThreads), 0, s,
                           (h16 *)Q, q_cols, (h16 *)K, k_cols, start_pos, head_dim, (const h16x2 *)table);
        AESIR_LAUNCH_CHECK("rope_vec_kernel");
        return AESIR_OK;
    }
    const int64_t total = q_rows * (q_cols / 2 + k_cols / 2);
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(total, kEThreads)), dim3(kEThreads), 0, s, (h16 *)Q, q_rows,
                       q_cols, (h16 *)K, k_cols, start_pos, head_dim, (const h16x2 *)table);
    AESIR_LAUNCH_CHECK("rope_kernel");
    return AESIR_OK;
}

// ------------------------------------------------------------------ silu / swiglu / residual
__global__ __launch_bounds__(kEThreads) void silu_kernel(h16 *__restrict__ T, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kEThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kEThreads)
        T[i] = silu_h(T[i]);
}

// silu(gate) in place, then up = f16(up * gate) (inference.mojo:258-260).
__global__ __launch_bounds__(kEThreads) void swiglu_kernel(h16 *__restrict__ up, h16 *__restrict__ gate, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kEThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kEThreads) {
        const h16 g = silu_h(gate[i]);
        gate[i] = g;
        up[i] = hmul(up[i], g);
    }
}

__global__ __launch_bounds__(kEThreads) void residual_kernel(h16 *__restrict__ x, const h16 *__restrict__ r, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kEThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kEThreads)
        x[i] = hadd(x[i], r[i]);
}

int32_t launch_silu(hipStream_t s, void *T, int64_t n) {
    hipLaunchKernelGGL(silu_kernel, dim3(grid_for(n, kEThreads)), dim3(kEThreads), 0, s, (h16 *)T, n);
    AESIR_LAUNCH_CHECK("silu_kernel");
    return AESIR_OK;
}

int32_t launch_swiglu(hipStream_t s, void *up, void *gate, int64_t n) {
    hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for(n, kEThreads)), dim3(kEThreads), 0, s, (h16 *)up, (h16 *)gate, n);
    AESIR_LAUNCH_CHECK("swiglu_kernel");
    return AESIR_OK;
}

int32_t launch_residual_add(hipStream_t s, void *x, const void *r, int64_t n) {
    hipLaunchKernelGGL(residual_kernel, dim3(grid_for(n, kEThreads)), dim3(kEThreads), 0, s, (h16 *)x, (const h16 *)r, n);
    AESIR_LAUNCH_CHECK("residual_kernel");
    return AESIR_OK;
}

// ------------------------------------------------------------------ embedding / KV append
// x = table[token] (inference.mojo:461-467); the token comes from `state` when given (graph replay).
__global__ __launch_bounds__(kEThreads) void embed_kernel(const h16 *__restrict__ table, int64_t dim, int64_t token,
                                                          const DecodeState *state, h16 *__restrict__ x) {
    const int64_t tok = state ? state->token : token;
    const h16 *row = table + tok * dim;
    for (int64_t i = threadIdx.x; i < dim; i += kEThreads) x[i] = row[i];
}

int32_t launch_embed(hipStream_t s, const void *table, int64_t dim, int64_t token, const DecodeState *state, void *x) {
    hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(kEThreads), 0, s, (const h16 *)table, dim, token, state, (h16 *)x);
    AESIR_LAUNCH_CHECK("embed_kernel");
    return AESIR_OK;
}

__global__ __launch_bounds__(kEThreads) void kv_append_kernel(h16 *__restrict__ kc, h16 *__restrict__ vc,
                                                              const h16 *__restrict__ k, const h16 *__restrict__ v,
                                                              int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kEThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kEThreads) {
        kc[i] = k[i];
        vc[i] = v[i];
    }
}

int32_t launch_kv_append(hipStream_t s, void *kc, void *vc, const void *k, const void *v, int64_t n) {
    hipLaunchKernelGGL(kv_append_kernel, dim3(grid_for(n, kEThreads)), dim3(kEThreads), 0, s, (h16 *)kc, (h16 *)vc,
                       (const h16 *)k, (const h16 *)v, n);
    AESIR_LAUNCH_CHECK("kv_append_kernel");
    return AESIR_OK;
}

// ------------------------------------------------------------------ seeded init
// Counter-based normal: element i of stream (seed, stream) from two SplitMix64-mixer outputs
// (the RuneRNG mixer of sampler.mojo:34-37) and Box-Muller in f64, rounded to f32 then f16.

// Element i (row i / cols, column i % cols) lands at dst[(i / cols) * dst_stride + i % cols], so a
// tensor can be generated straight into an interleaved layout.
__global__ __launch_bounds__(kEThreads) void fill_normal_kernel(h16 *__restrict__ dst, int64_t n, int64_t cols,
                                                                int64_t dst_stride, uint64_t base, double mean,
                                                                double std) {
    for (int64_t i = (int64_t)blockIdx.x * kEThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kEThreads) {
        const uint64_t a = mix64(base + (uint64_t)(2 * i + 1) * kGolden);
        const uint64_t b = mix64(base + (uint64_t)(2 * i + 2) * kGolden);
        const double u1 = (double)((a >> 40) + 1) * (1.0 / 16777216.0);
        const double u2 = (double)(b >> 40) * (1.0 / 16777216.0);
        const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        dst[(i / cols) * dst_stride + i % cols] = (h16)(float)(mean + std * z);
    }
}

int32_t launch_fill_normal(hipStream_t s, void *dst, int64_t n, int64_t cols, int64_t dst_stride, uint64_t seed,
                           uint64_t stream, float mean, float std) {
    const uint64_t base = mix64(seed ^ mix64(stream + kGolden));
    hipLaunchKernelGGL(fill_normal_kernel, dim3(grid_for(n, kEThreads * 8)), dim3(kEThreads), 0, s, (h16 *)dst, n,
                       cols, dst_stride, base, (double)mean, (double)std);
    AESIR_LAUNCH_CHECK("fill_normal_kernel");
    return AESIR_OK;
}

// Q8_0 init: quant i (row i / cols, column i % cols) uniform in [-127, 127] (standard deviation
// 73.3); block j's scale uniform in [0.5, 1.5) * std / 64, rounded to f16, so the weights have a
// standard deviation near std. Counter streams as in fill_normal_kernel (quants from odd
// counters, scales from even ones).
__global__ __launch_bounds__(kEThreads) void fill_q8_0_kernel(int8_t *__restrict__ q, int64_t q_stride,
                                                              h16 *__restrict__ d, int64_t d_stride, int64_t rows,
                                                              int64_t cols, uint64_t base, double dscale) {
    const int64_t nb = cols / 32, n = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * kEThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kEThreads) {
        const uint64_t a = mix64(base + (uint64_t)(2 * i + 1) * kGolden);
        q[(i / cols) * q_stride + i % cols] = (int8_t)((int)((a >> 32) % 255u) - 127);
        if (i % 32 == 0) {
            const int64_t j = i / 32;
            const uint64_t b = mix64(base + (uint64_t)(2 * j + 2) * kGolden);
            const double u = (double)(b >> 40) * (1.0 / 16777216.0);
            d[(j / nb) * d_stride + j % nb] = (h16)(float)((0.5 + u) * dscale);
        }
    }
}

int32_t launch_fill_q8_0(hipStream_t s, void *q, int64_t q_stride, void *d, int64_t d_stride, int64_t rows,
                         int64_t cols, uint64_t seed, uint64_t stream, float std) {
    if (cols % 32 != 0) return fail(AESIR_ERR_SHAPE, "fill_q8_0: columns must be a multiple of 32");
    const uint64_t base = mix64(seed ^ mix64(stream + kGolden));
    hipLaunchKernelGGL(fill_q8_0_kernel, dim3(grid_for(rows * cols, kEThreads * 8)), dim3(kEThreads), 0, s,
                       (int8_t *)q, q_stride, (h16 *)d, d_stride, rows, cols, base, (double)std / 64.0);
    AESIR_LAUNCH_CHECK("fill_q8_0_kernel");
    return AESIR_OK;
}

__global__ __launch_bounds__(kEThreads) void f32_to_f16_kernel(const float *__restrict__ src, h16 *__restrict__ dst,
                                                               int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kEThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kEThreads)
        dst[i] = (h16)src[i];
}

int32_t launch_f32_to_f16(hipStream_t s, const float *src, void *dst, int64_t n) {
    hipLaunchKernelGGL(f32_to_f16_kernel, dim3(grid_for(n, kEThreads)), dim3(kEThreads), 0, s, src, (h16 *)dst, n);
    AESIR_LAUNCH_CHECK("f32_to_f16_kernel");
    return AESIR_OK;
}

}  // namespace aesir
