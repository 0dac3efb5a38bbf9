// Device-side helpers for gfx950 (CDNA4): binary16 arithmetic with the reference's rounding
// points, 16-byte vector loads and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace aesir {

typedef _Float16 h16;
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));

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

// ------------------------------------------------------------------ counter-based generator
// SplitMix64's finalizer; synthetic weights draw element i of a stream from mix64(base + i * kGolden).
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ULL;

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

// D = A B + C on one 16 x 16 x 32 f16 tile (v_mfma_f32_16x16x32_f16). Lane l holds A row l % 16
// and B column l % 16, each with k = 8 (l / 16) .. + 7 (8 halves), and D rows 4 (l / 16) + e,
// column l % 16, in element e.
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h16x8, a), __builtin_bit_cast(h16x8, b), c, 0, 0,
                                                  0);
}

// ------------------------------------------------------------------ reductions
// Cross-lane steps without LDS: DPP row patterns for partners within a 16-lane row, and gfx950's
// v_permlane16_swap / v_permlane32_swap for partners 16 and 32 lanes away. Every step combines a
// lane with a partner whose position in the reduction tree is symmetric (x ^ 1, x ^ 2, 7 - x in
// each 8-lane half, 15 - x in each row, x ^ 16, x ^ 32), so after the steps of a group every lane
// of the group holds the same value. The patterns read every lane of the group: call them with
// the whole wave active.
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // 7 - x within each 8-lane half row
constexpr int kDppMirror = 0x140;     // 15 - x within each 16-lane row

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// (value of a in the lower lane of each pair, value of b in the upper lane), for lane pairs
// (x, x + 16) in every 32 lanes (D = 16) or (x, x + 32) (D = 32); the sum of the two results is
// a(lower) + a(upper) in lower lanes and b(lower) + b(upper) in upper lanes.
template <int D>
__device__ __forceinline__ float swap_pair_sum(float a, float b) {
    const unsigned ua = __builtin_bit_cast(unsigned, a), ub = __builtin_bit_cast(unsigned, b);
    if constexpr (D == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(ua, ub, false, false);
        return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(ua, ub, false, false);
        return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
    }
}
template <int D>
__device__ __forceinline__ float swap_pair_max(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    if constexpr (D == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
    }
}

// Sum / max over aligned groups of L lanes (L = 1, 2, 4, ..., 64); every lane of a group gets it.
template <int L>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (L >= 2) v += dpp_f<kDppXor1>(v);
    if constexpr (L >= 4) v += dpp_f<kDppXor2>(v);
    if constexpr (L >= 8) v += dpp_f<kDppHalfMirror>(v);
    if constexpr (L >= 16) v += dpp_f<kDppMirror>(v);
    if constexpr (L >= 32) v = swap_pair_sum<16>(v, v);
    if constexpr (L >= 64) v = swap_pair_sum<32>(v, v);
    return v;
}
template <int L>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (L >= 2) v = fmaxf(v, dpp_f<kDppXor1>(v));
    if constexpr (L >= 4) v = fmaxf(v, dpp_f<kDppXor2>(v));
    if constexpr (L >= 8) v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    if constexpr (L >= 16) v = fmaxf(v, dpp_f<kDppMirror>(v));
    if constexpr (L >= 32) v = swap_pair_max<16>(v);
    if constexpr (L >= 64) v = swap_pair_max<32>(v);
    return v;
}
__device__ __forceinline__ float wave_sum(float v) { return group_sum<kWave>(v); }
__device__ __forceinline__ float wave_max(float v) { return group_max<kWave>(v); }

// Minimum of an int over the wave (the same halving steps as group_max); every lane gets it.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ int wave_min_i(int v) {
    v = min(v, dpp_i<kDppXor1>(v));
    v = min(v, dpp_i<kDppXor2>(v));
    v = min(v, dpp_i<kDppHalfMirror>(v));
    v = min(v, dpp_i<kDppMirror>(v));
    const auto r16 = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    v = min((int)r16[0], (int)r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    return min((int)r32[0], (int)r32[1]);
}

// Reduces R per-lane partial sums across the wave by recursive halving: after the call, every
// lane holds the full wave sum of row (lane / (64 / R)) in v[0]. R is a power of two <= 64.
// Halving steps pair lanes 32 apart, then 16, 8 (15 - x), 4 (7 - x), 2, 1; at each step the
// lane whose partner bit is set keeps the upper half of its live rows.
template <int R>
__device__ __forceinline__ float wave_multi_sum(float (&v)[R], int lane) {
    int live = R;
    auto halve_swap = [&](auto dist) {
        constexpr int D = decltype(dist)::value;
        if (live > 1) {
            const int half = live >> 1;
#pragma unroll
            for (int r = 0; r < R / 2; r++)
                if (r < half) v[r] = swap_pair_sum<D>(v[r], v[r + half]);
            live = half;
        } else {
            v[0] = swap_pair_sum<D>(v[0], v[0]);
        }
    };
    halve_swap(std::integral_constant<int, 32>{});
    halve_swap(std::integral_constant<int, 16>{});
    auto halve_dpp = [&](auto ctrl, int bit) {
        constexpr int C = decltype(ctrl)::value;
        if (live > 1) {
            const int half = live >> 1;
            const bool upper = (lane & bit) != 0;
#pragma unroll
            for (int r = 0; r < R / 2; r++) {
                if (r < half) {
                    const float keep = upper ? v[r + half] : v[r];
                    const float give = upper ? v[r] : v[r + half];
                    v[r] = keep + dpp_f<C>(give);
                }
            }
            live = half;
        } else {
            v[0] += dpp_f<C>(v[0]);
        }
    };
    halve_dpp(std::integral_constant<int, kDppMirror>{}, 8);
    halve_dpp(std::integral_constant<int, kDppHalfMirror>{}, 4);
    halve_dpp(std::integral_constant<int, kDppXor2>{}, 2);
    halve_dpp(std::integral_constant<int, kDppXor1>{}, 1);
    return v[0];
}

// Workgroup-wide sum for blockDim.x == 64 * NW; `red` is shared scratch of >= NW floats.
// REUSE = false: the caller never writes `red` again, so the barrier that would protect it from
// the next use is left out.
template <int NW, bool REUSE = true>
__device__ __forceinline__ float block_sum(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; w++) s += red[w];
    if (REUSE) __syncthreads();
    return s;
}

}  // namespace aesir
