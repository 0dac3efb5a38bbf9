// Device-side helpers for gfx950 (CDNA4): binary16 arithmetic with the reference's rounding
// points, 16-byte vector loads and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace aesir {

typedef _Float16 h16;
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ------------------------------------------------------------------ binary16 ops
// Each op is evaluated in f32 and rounded once to f16 (v_cvt_f16_f32, round to nearest even),
// which equals the correctly rounded binary16 result for + - * /. The library is built with
// -ffp-contract=off, so no multiply-add is fused across these roundings.
__device__ __forceinline__ h16 hmul(h16 a, h16 b) { return (h16)((float)a * (float)b); }
__device__ __forceinline__ h16 hadd(h16 a, h16 b) { return (h16)((float)a + (float)b); }
__device__ __forceinline__ h16 hsub(h16 a, h16 b) { return (h16)((float)a - (float)b); }
__device__ __forceinline__ h16 hdiv(h16 a, h16 b) { return (h16)((float)a / (float)b); }

__device__ __forceinline__ h16 bits_to_h(uint16_t b) { return __builtin_bit_cast(h16, b); }
__device__ __forceinline__ uint16_t h_to_bits(h16 h) { return __builtin_bit_cast(uint16_t, h); }

// silu (compute.mojo:2113-2126) on one f16 value: x * (1 / (1 + exp(-x))), every op in f16.
// exp is evaluated in f64 and rounded to f32 then f16, i.e. the correctly rounded f32 exp
// followed by the f16 rounding that the reference applies to its f16 exp.
__device__ __forceinline__ h16 silu_h(h16 x) {
    const h16 one = (h16)1.0f;
    h16 e = (h16)(float)exp(-(double)(float)x);
    h16 sig = hdiv(one, hadd(one, e));
    return hmul(x, sig);
}

// ------------------------------------------------------------------ vector loads
__device__ __forceinline__ u32x4 ld16(const void *p) { return *reinterpret_cast<const u32x4 *>(p); }
// Streaming weight load: non-temporal hint so single-use weights do not evict reused data.
__device__ __forceinline__ u32x4 ld16_stream(const void *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}
__device__ __forceinline__ void st16(void *p, u32x4 v) { *reinterpret_cast<u32x4 *>(p) = v; }

__device__ __forceinline__ h16x2 as_h2(unsigned int u) { return __builtin_bit_cast(h16x2, u); }
__device__ __forceinline__ unsigned int h2_bits(h16x2 h) { return __builtin_bit_cast(unsigned int, h); }

// acc + sum of the 8 f16 products of two 16-byte vectors (v_dot2_f32_f16, f32 accumulate).
// f16(q_j * d) of the four int8 quants in w (byte j = quant j), as two f16 pairs (quants 0, 1 and
// 2, 3). int8 -> f16 is exact through the exponent trick (byte ^ 0x80 placed under the f16
// exponent of 1024 reads 1152 + q; subtracting 1152 is exact); the packed f16 multiply by d
// rounds once, as the f16 product f16(q) * d does.
__device__ __forceinline__ void dequant_q8x4(unsigned w, h16 d, unsigned &lo, unsigned &hi) {
    const unsigned u = w ^ 0x80808080u;
    const h16x2 bias = {(h16)1152.0f, (h16)1152.0f}, dd = {d, d};
    lo = h2_bits((as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias) * dd);
    hi = h2_bits((as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias) * dd);
}

__device__ __forceinline__ float dot8(u32x4 a, u32x4 b, float acc) {
    acc = __builtin_amdgcn_fdot2(as_h2(a.x), as_h2(b.x), acc, false);
    acc = __builtin_amdgcn_fdot2(as_h2(a.y), as_h2(b.y), acc, false);
    acc = __builtin_amdgcn_fdot2(as_h2(a.z), as_h2(b.z), acc, false);
    acc = __builtin_amdgcn_fdot2(as_h2(a.w), as_h2(b.w), acc, false);
    return acc;
}

// ------------------------------------------------------------------ reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Reduces R per-lane partial sums across the wave by recursive halving: after the call, every
// lane holds the full wave sum of row (lane / (64 / R)) in v[0]. R is a power of two <= 64.
template <int R>
__device__ __forceinline__ float wave_multi_sum(float (&v)[R], int lane) {
    int live = R;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        if (live > 1) {
            const int half = live >> 1;
            const bool upper = (lane & o) != 0;
#pragma unroll
            for (int r = 0; r < R / 2; r++) {
                if (r < half) {
                    float keep = upper ? v[r + half] : v[r];
                    float give = upper ? v[r] : v[r + half];
                    v[r] = keep + __shfl_xor(give, o, kWave);
                }
            }
            live = half;
        } else {
            v[0] += __shfl_xor(v[0], o, kWave);
        }
    }
    return v[0];
}

// Workgroup-wide sum for blockDim.x == 64 * NW; `red` is shared scratch of >= NW floats.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; w++) s += red[w];
    __syncthreads();
    return s;
}

}  // namespace aesir
