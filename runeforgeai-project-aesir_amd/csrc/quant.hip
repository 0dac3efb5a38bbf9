// 4-bit and K-quant weights on gfx950: GGML Q4_0 (with the reference's gemm_q4_0 rounding,
// core/compute.mojo:876-912) and GGML's Q4_K / Q6_K super-blocks.
//
// GGUF stores these as packed blocks of 18, 144 and 210 bytes whose nibble order suits a CPU
// loop, not a wave: the bytes of one block are read by one lane, and 210 is not even 4-byte
// aligned. At upload every matrix is repacked (QFMat in kernels.hpp) into records of 16 weights:
// 8 nibble bytes per record, arranged so that one AND-OR with 0x64006400 turns a nibble pair into
// the f16 pair (1024 + q_a, 1024 + q_b) for weights (a, a + 2), plus small planes of per-block
// scales. A GEMV lane multiplies one record per row and slab (k = 16 t + 4096 i): an 8-byte
// nibble load per row, x held in registers in the matching pair order.
//
// Arithmetic per type:
//   Q4_0  w = f16(f16(q - 8) * d), the reference's dequantize_q4_0 (compute.mojo:266-280): the
//         pair (1024 + q) - 1032 is exact, the packed f16 multiply by d rounds once; then f32
//         v_dot2_f32_f16 accumulation as in the F16 path.
//   Q4_K  w = (d * sc) * q - dmin * m, GGML's value in f32. Per record (16 weights of one 32-weight
//         sub-block): S = sum x q with q exact in f16, X = sum x; contribution (d sc) S - (dmin m) X
//         in f32.
//   Q6_K  w = (d * sc) * (q - 32): S = sum x (q - 32) with the 6-bit value exact in f16
//         ((1024 + q) - 1056), contribution (d sc) S in f32.
// The K-quant dot products therefore use the f32 weights GGML defines, not f16-rounded ones.
#include <atomic>

#include "device.hpp"
#include "gemv_common.hpp"
#include "kernels.hpp"

namespace aesir {

constexpr int kRec = 16;                                 // weights per record
constexpr int64_t kQfSlab = (int64_t)kThreads * kRec;    // k covered by one workgroup pass
constexpr unsigned kMagic = 0x64006400u;                 // f16 1024 in both halves
constexpr int kQfRows = 4;                               // rows per group of the decode GEMVs
constexpr int kQfMaxSlabs = 7;                           // K <= 28672

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

bool qf_type(int32_t t) { return t == AESIR_GGML_Q4_0 || t == AESIR_GGML_Q4_K || t == AESIR_GGML_Q6_K; }

// Bit position of the high 2 bits of record weight i in the Q6_K hb word: weights a and a + 2
// of nibble pair f (a = {0, 1, 4, 5, 8, 9, 12, 13}[f]) sit 16 bits apart at bits 2 f, 2 f + 16.
__host__ __device__ __forceinline__ int qf_hb_pos(int i) { return 16 * ((i >> 1) & 1) + 2 * (2 * (i >> 2) + (i & 1)); }

// ------------------------------------------------------------------ one record

template <int T>
struct QRec;
template <>
struct QRec<AESIR_GGML_Q4_0> {
    u32x2 nib;
    h16 d;
};
template <>
struct QRec<AESIR_GGML_Q4_K> {
    u32x2 nib;
    unsigned scm;  // scale | min << 8
    unsigned dd;   // f16 d | f16 dmin << 16
};
template <>
struct QRec<AESIR_GGML_Q6_K> {
    u32x2 nib;
    unsigned hb;
    int sc;
    h16 d;
};

// Record `rec` of plane row `prow` (the row index in plane rows, i.e. already scaled by step).
template <int T>
__device__ __forceinline__ QRec<T> qf_load(const QFMat &w, int64_t prow, int64_t rec, int64_t K) {
    QRec<T> q;
    q.nib = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>((const uint8_t *)w.nib + prow * (K / 2)) + rec);
    if constexpr (T == AESIR_GGML_Q4_0) {
        q.d = reinterpret_cast<const h16 *>(w.s0)[prow * (K / 32) + rec / 2];
    } else if constexpr (T == AESIR_GGML_Q4_K) {
        q.scm = reinterpret_cast<const uint16_t *>(w.s0)[prow * (K / 32) + rec / 2];
        q.dd = reinterpret_cast<const uint32_t *>(w.s1)[prow * (K / 256) + rec / 16];
    } else {
        q.hb = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(w.hb) + prow * (K / 16) + rec);
        q.sc = reinterpret_cast<const int8_t *>(w.s0)[prow * (K / 16) + rec];
        q.d = reinterpret_cast<const h16 *>(w.s1)[prow * (K / 256) + rec / 16];
    }
    return q;
}

// f16 pair (1024 + q_a, 1024 + q_b) of nibble pair f (weights a, a + 2 of the record), with the
// Q6_K high bits OR-ed in when given.
__device__ __forceinline__ unsigned qf_pair(u32x2 nib, int f) {
    const int sh = (f & 1) * 8 + (f >> 2) * 4;
    return (((f >> 1) & 1 ? nib.y : nib.x) >> sh) & 0x000F000Fu;
}
__device__ __forceinline__ unsigned qf_hb_pair(unsigned hb, int f) {
    const int s = 4 - 2 * f;
    return (s >= 0 ? hb << s : hb >> -s) & 0x00300030u;
}

// x of one record in pair order: xp[f] = (x[a_f], x[a_f + 2]) from the natural chunks x[0..7],
// x[8..15].
__device__ __forceinline__ void qf_perm_x(const u32x4 (&x)[2], unsigned (&xp)[8]) {
#pragma unroll
    for (int c = 0; c < 2; c++) {
        xp[4 * c + 0] = __builtin_amdgcn_perm(x[c].y, x[c].x, 0x05040100u);
        xp[4 * c + 1] = __builtin_amdgcn_perm(x[c].y, x[c].x, 0x07060302u);
        xp[4 * c + 2] = __builtin_amdgcn_perm(x[c].w, x[c].z, 0x05040100u);
        xp[4 * c + 3] = __builtin_amdgcn_perm(x[c].w, x[c].z, 0x07060302u);
    }
}

// Exact f16 pairs of the record's quantized values, pair order: Q4_0 q - 8, Q4_K q, Q6_K q - 32.
template <int T>
__device__ __forceinline__ h16x2 qf_qpair(const QRec<T> &q, int f) {
    if constexpr (T == AESIR_GGML_Q4_0) {
        const h16x2 bias = {(h16)1032.0f, (h16)1032.0f};
        return as_h2(qf_pair(q.nib, f) | kMagic) - bias;
    } else if constexpr (T == AESIR_GGML_Q4_K) {
        const h16x2 bias = {(h16)1024.0f, (h16)1024.0f};
        return as_h2(qf_pair(q.nib, f) | kMagic) - bias;
    } else {
        const h16x2 bias = {(h16)1056.0f, (h16)1056.0f};
        return as_h2(qf_pair(q.nib, f) | qf_hb_pair(q.hb, f) | kMagic) - bias;
    }
}

// acc + this record's share of the row's dot product (xs: sum of the record's 16 x values).
template <int T>
__device__ __forceinline__ float qf_dot(const QRec<T> &q, const unsigned (&xp)[8], float xs, float acc) {
    if constexpr (T == AESIR_GGML_Q4_0) {
        const h16x2 dd = {q.d, q.d};
#pragma unroll
        for (int f = 0; f < 8; f++) acc = __builtin_amdgcn_fdot2(qf_qpair(q, f) * dd, as_h2(xp[f]), acc, false);
        return acc;
    } else {
        float S = 0.0f;
#pragma unroll
        for (int f = 0; f < 8; f++) S = __builtin_amdgcn_fdot2(qf_qpair(q, f), as_h2(xp[f]), S, false);
        if constexpr (T == AESIR_GGML_Q4_K) {
            const float d = (float)bits_to_h((uint16_t)(q.dd & 0xffffu)), dm = (float)bits_to_h((uint16_t)(q.dd >> 16));
            const float a = d * (float)(q.scm & 0xffu), b = dm * (float)(q.scm >> 8);
            return acc + (a * S - b * xs);
        } else {
            return acc + ((float)q.d * (float)q.sc) * S;
        }
    }
}

// The record's 16 weights as f16 in natural order (o[0]: weights 0..7, o[1]: 8..15):
// Q4_0 f16((q - 8) d); Q4_K f16((d sc) q - dmin m); Q6_K f16((d sc) (q - 32)) with the products
// in f32 (GGML's f32 value, then one rounding to f16).
template <int T>
__device__ __forceinline__ void qf_deq16(const QRec<T> &q, u32x4 (&o)[2]) {
    unsigned wp[8];
#pragma unroll
    for (int f = 0; f < 8; f++) {
        const h16x2 v = qf_qpair(q, f);
        if constexpr (T == AESIR_GGML_Q4_0) {
            const h16x2 dd = {q.d, q.d};
            wp[f] = h2_bits(v * dd);
        } else if constexpr (T == AESIR_GGML_Q4_K) {
            const float d = (float)bits_to_h((uint16_t)(q.dd & 0xffffu)), dm = (float)bits_to_h((uint16_t)(q.dd >> 16));
            const float a = d * (float)(q.scm & 0xffu), b = dm * (float)(q.scm >> 8);
            h16x2 r;
            r.x = (h16)(a * (float)v.x - b);
            r.y = (h16)(a * (float)v.y - b);
            wp[f] = h2_bits(r);
        } else {
            const float a = (float)q.d * (float)q.sc;
            h16x2 r;
            r.x = (h16)(a * (float)v.x);
            r.y = (h16)(a * (float)v.y);
            wp[f] = h2_bits(r);
        }
    }
#pragma unroll
    for (int c = 0; c < 2; c++) {
        o[c].x = __builtin_amdgcn_perm(wp[4 * c + 1], wp[4 * c + 0], 0x05040100u);
        o[c].y = __builtin_amdgcn_perm(wp[4 * c + 1], wp[4 * c + 0], 0x07060302u);
        o[c].z = __builtin_amdgcn_perm(wp[4 * c + 3], wp[4 * c + 2], 0x05040100u);
        o[c].w = __builtin_amdgcn_perm(wp[4 * c + 3], wp[4 * c + 2], 0x07060302u);
    }
}

// ------------------------------------------------------------------ repacking

// GGUF source of weight e of a row: its 4- or 6-bit value and block metadata.
template <int T>
__device__ __forceinline__ int gguf_q(const uint8_t *row, int64_t e) {
    if constexpr (T == AESIR_GGML_Q4_0) {
        const uint8_t *blk = row + (e / 32) * 18;
        const int i = (int)(e % 32);
        return i < 16 ? (blk[2 + i] & 15) : (blk[2 + i - 16] >> 4);
    } else if constexpr (T == AESIR_GGML_Q4_K) {
        const uint8_t *qs = row + (e / 256) * 144 + 16;
        const int i = (int)(e % 256), g = i / 64, l = i % 64;
        return l < 32 ? (qs[32 * g + l] & 15) : (qs[32 * g + l - 32] >> 4);
    } else {
        const uint8_t *blk = row + (e / 256) * 210;
        const int i = (int)(e % 256), h = i / 128, t = i % 128, grp = t / 32, l = t % 32;
        const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
        const int lo = grp & 1 ? ql[l + 32] : ql[l];
        const int nib = grp < 2 ? (lo & 15) : (lo >> 4);
        return nib | (((qh[l] >> (2 * grp)) & 3) << 4);
    }
}

// 6-bit scale and min of Q4_K sub-block j (GGML's packing of scales[12]).
__device__ __forceinline__ void q4k_scale_min(const uint8_t *sc, int j, int &s, int &m) {
    if (j < 4) {
        s = sc[j] & 63;
        m = sc[j + 4] & 63;
    } else {
        s = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4);
        m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}

__device__ __forceinline__ uint8_t *plane_row(const void *p, int32_t type, int plane, int64_t prow, int64_t K) {
    return (uint8_t *)p + prow * qf_plane_row_bytes(type, plane, K);
}

// One thread per record: GGUF blocks -> nibble record (+ hb word) and, from the record that
// starts a block, its metadata.
template <int T>
__global__ __launch_bounds__(256) void qf_repack_kernel(const uint8_t *__restrict__ blocks, int64_t rows, int64_t K,
                                                        QFMat dst, int64_t step) {
    const int64_t recs = K / kRec;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= rows * recs) return;
    const int64_t r = gid / recs, rec = gid % recs, k = rec * kRec;
    const int64_t bpr = T == AESIR_GGML_Q4_0 ? K / 32 * 18 : T == AESIR_GGML_Q4_K ? K / 256 * 144 : K / 256 * 210;
    const uint8_t *src = blocks + r * bpr;
    const int64_t prow = r * step;
    int q[kRec];
#pragma unroll
    for (int i = 0; i < kRec; i++) q[i] = gguf_q<T>(src, k + i);
    unsigned nib[2] = {0u, 0u}, hb = 0u;
#pragma unroll
    for (int j = 0; j < 8; j++) nib[j >> 2] |= (unsigned)((q[j] & 15) | ((q[8 + j] & 15) << 4)) << (8 * (j & 3));
    if constexpr (T == AESIR_GGML_Q6_K) {
#pragma unroll
        for (int i = 0; i < kRec; i++) hb |= (unsigned)(q[i] >> 4) << qf_hb_pos(i);
        reinterpret_cast<uint32_t *>(plane_row(dst.hb, T, 1, prow, K))[rec] = hb;
    }
    reinterpret_cast<u32x2 *>(plane_row(dst.nib, T, 0, prow, K))[rec] = u32x2{nib[0], nib[1]};
    if constexpr (T == AESIR_GGML_Q4_0) {
        if (rec % 2 == 0) {
            const uint8_t *blk = src + (k / 32) * 18;
            reinterpret_cast<uint16_t *>(plane_row(dst.s0, T, 2, prow, K))[k / 32] = (uint16_t)(blk[0] | (blk[1] << 8));
        }
    } else if constexpr (T == AESIR_GGML_Q4_K) {
        const uint8_t *blk = src + (k / 256) * 144;
        if (rec % 2 == 0) {
            int s, m;
            q4k_scale_min(blk + 4, (int)((k % 256) / 32), s, m);
            reinterpret_cast<uint16_t *>(plane_row(dst.s0, T, 2, prow, K))[k / 32] = (uint16_t)(s | (m << 8));
        }
        if (rec % 16 == 0)
            reinterpret_cast<uint32_t *>(plane_row(dst.s1, T, 3, prow, K))[k / 256] =
                (uint32_t)blk[0] | ((uint32_t)blk[1] << 8) | ((uint32_t)blk[2] << 16) | ((uint32_t)blk[3] << 24);
    } else {
        const uint8_t *blk = src + (k / 256) * 210;
        reinterpret_cast<int8_t *>(plane_row(dst.s0, T, 2, prow, K))[k / 16] = (int8_t)blk[192 + (k % 256) / 16];
        if (rec % 16 == 0)
            reinterpret_cast<uint16_t *>(plane_row(dst.s1, T, 3, prow, K))[k / 256] =
                (uint16_t)(blk[208] | (blk[209] << 8));
    }
}

// One thread per record: planes -> f16 weights (natural order).
template <int T>
__global__ __launch_bounds__(256) void qf_dequant_kernel(QFMat w, int64_t rows, int64_t K, int64_t step,
                                                         const int64_t *__restrict__ row_ids, h16 *__restrict__ out,
                                                         int64_t out_stride) {
    const int64_t recs = K / kRec;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= rows * recs) return;
    const int64_t r = gid / recs, rec = gid % recs;
    const int64_t src_row = row_ids ? row_ids[r] : r;
    u32x4 o[2];
    qf_deq16<T>(qf_load<T>(w, src_row * step, rec, K), o);
    h16 *dst = out + r * out_stride + rec * kRec;
    st16(dst, o[0]);
    st16(dst + 8, o[1]);
}

// One thread per record: uniform random values; scales chosen so that the weights have a
// standard deviation near `std` and a mean near 0.
template <int T>
__global__ __launch_bounds__(256) void qf_fill_kernel(QFMat w, int64_t rows, int64_t K, int64_t step, uint64_t base,
                                                      float std) {
    const int64_t recs = K / kRec;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= rows * recs) return;
    const int64_t r = gid / recs, rec = gid % recs, prow = r * step;
    const uint64_t a = mix64(base + (uint64_t)(2 * gid + 1) * kGolden);
    const uint64_t b = mix64(base + (uint64_t)(2 * gid + 2) * kGolden);
    reinterpret_cast<u32x2 *>(plane_row(w.nib, T, 0, prow, K))[rec] = u32x2{(unsigned)a, (unsigned)(a >> 32)};
    const float u = (float)(b >> 40) * (1.0f / 16777216.0f);  // [0, 1)
    if constexpr (T == AESIR_GGML_Q4_0) {
        // q - 8 uniform on [-8, 7]: standard deviation 4.61
        if (rec % 2 == 0) reinterpret_cast<h16 *>(plane_row(w.s0, T, 2, prow, K))[rec / 2] = (h16)((0.5f + u) * std / 4.61f);
    } else if constexpr (T == AESIR_GGML_Q4_K) {
        // sc in [4, 8], m = round(7.5 sc), dmin = d: w = d sc (q - 7.5) nearly, q uniform on [0, 15]
        if (rec % 2 == 0) {
            const int s = 4 + (int)((b >> 8) % 5), m = (int)(7.5f * (float)s + 0.5f);
            reinterpret_cast<uint16_t *>(plane_row(w.s0, T, 2, prow, K))[rec / 2] = (uint16_t)(s | (m << 8));
        }
        if (rec % 16 == 0) {
            const h16 d = (h16)((0.5f + u) * std / (6.0f * 4.61f));
            const uint32_t dv = h_to_bits(d);
            reinterpret_cast<uint32_t *>(plane_row(w.s1, T, 3, prow, K))[rec / 16] = dv | (dv << 16);
        }
    } else {
        // q - 32 uniform on [-32, 31]: standard deviation 18.5; sc in [16, 47]
        reinterpret_cast<uint32_t *>(plane_row(w.hb, T, 1, prow, K))[rec] = (uint32_t)(b >> 8);
        reinterpret_cast<int8_t *>(plane_row(w.s0, T, 2, prow, K))[rec] = (int8_t)(16 + (int)((b >> 4) % 32));
        if (rec % 16 == 0)
            reinterpret_cast<h16 *>(plane_row(w.s1, T, 3, prow, K))[rec / 16] = (h16)((0.5f + u) * std / (32.0f * 18.5f));
    }
}

static unsigned rec_grid(int64_t rows, int64_t K) { return (unsigned)((rows * (K / kRec) + 255) / 256); }

static int32_t qf_check(int32_t type, int64_t K, const char *name) {
    if (!qf_type(type)) return fail(AESIR_ERR_UNSUPPORTED, "%s: weight type %d is not Q4_0, Q4_K or Q6_K", name, (int)type);
    const int64_t blk = type == AESIR_GGML_Q4_0 ? 32 : 256;
    if (K <= 0 || K % blk != 0)
        return fail(AESIR_ERR_SHAPE, "%s: row length %lld is not a multiple of the %lld-weight block", name, (long long)K,
                    (long long)blk);
    return AESIR_OK;
}

int32_t launch_qf_repack(hipStream_t s, int32_t type, const void *blocks, int64_t rows, int64_t K, const QFMat &dst,
                         int64_t step) {
    AESIR_TRY(qf_check(type, K, "repack"));
    if (rows <= 0) return AESIR_OK;
    const unsigned g = rec_grid(rows, K);
    if (type == AESIR_GGML_Q4_0)
        hipLaunchKernelGGL(qf_repack_kernel<AESIR_GGML_Q4_0>, dim3(g), dim3(256), 0, s, (const uint8_t *)blocks, rows, K, dst, step);
    else if (type == AESIR_GGML_Q4_K)
        hipLaunchKernelGGL(qf_repack_kernel<AESIR_GGML_Q4_K>, dim3(g), dim3(256), 0, s, (const uint8_t *)blocks, rows, K, dst, step);
    else
        hipLaunchKernelGGL(qf_repack_kernel<AESIR_GGML_Q6_K>, dim3(g), dim3(256), 0, s, (const uint8_t *)blocks, rows, K, dst, step);
    AESIR_LAUNCH_CHECK("qf_repack_kernel");
    return AESIR_OK;
}

int32_t launch_qf_dequant(hipStream_t s, const QFMat &w, int64_t rows, int64_t K, int64_t step,
                          const int64_t *row_ids, void *out, int64_t out_stride) {
    AESIR_TRY(qf_check(w.type, K, "dequant"));
    if (rows <= 0) return AESIR_OK;
    const unsigned g = rec_grid(rows, K);
    if (w.type == AESIR_GGML_Q4_0)
        hipLaunchKernelGGL(qf_dequant_kernel<AESIR_GGML_Q4_0>, dim3(g), dim3(256), 0, s, w, rows, K, step, row_ids, (h16 *)out, out_stride);
    else if (w.type == AESIR_GGML_Q4_K)
        hipLaunchKernelGGL(qf_dequant_kernel<AESIR_GGML_Q4_K>, dim3(g), dim3(256), 0, s, w, rows, K, step, row_ids, (h16 *)out, out_stride);
    else
        hipLaunchKernelGGL(qf_dequant_kernel<AESIR_GGML_Q6_K>, dim3(g), dim3(256), 0, s, w, rows, K, step, row_ids, (h16 *)out, out_stride);
    AESIR_LAUNCH_CHECK("qf_dequant_kernel");
    return AESIR_OK;
}

int32_t launch_qf_fill_random(hipStream_t s, const QFMat &w, int64_t rows, int64_t K, int64_t step, uint64_t seed,
                              uint64_t stream, float std) {
    AESIR_TRY(qf_check(w.type, K, "fill"));
    if (rows <= 0) return AESIR_OK;
    const uint64_t base = mix64(seed ^ mix64(stream + kGolden));
    const unsigned g = rec_grid(rows, K);
    if (w.type == AESIR_GGML_Q4_0)
        hipLaunchKernelGGL(qf_fill_kernel<AESIR_GGML_Q4_0>, dim3(g), dim3(256), 0, s, w, rows, K, step, base, std);
    else if (w.type == AESIR_GGML_Q4_K)
        hipLaunchKernelGGL(qf_fill_kernel<AESIR_GGML_Q4_K>, dim3(g), dim3(256), 0, s, w, rows, K, step, base, std);
    else
        hipLaunchKernelGGL(qf_fill_kernel<AESIR_GGML_Q6_K>, dim3(g), dim3(256), 0, s, w, rows, K, step, base, std);
    AESIR_LAUNCH_CHECK("qf_fill_kernel");
    return AESIR_OK;
}

// ------------------------------------------------------------------ decode GEMV

// x source: x itself, or (layer 0) row token->token of the repacked embedding table, dequantized
// in registers, with workgroup 0 writing the row to xcopy (the residual stream).
struct QFXSrc {
    const h16 *x;
    QFMat emb;
    const DecodeState *token;
    h16 *xcopy;
};

// Thread t multiplies record t + 256 i (k = 16 t + 4096 i, NS slabs) of ROWS rows per group, G
// groups per workgroup; x stays in registers (RMS-normalized once, then put in pair order); the
// weight requests run D (group, slab) steps ahead through a register ring. Same structure and
// epilogues as the Q8_0 GEMV.
template <int T, int ROWS, int NS, int G, bool NORM, class Epi>
__global__ __launch_bounds__(kThreads) void gemv_qf_kernel(QFMat w, int64_t N, int64_t K, QFXSrc src,
                                                           const h16 *__restrict__ nw, float eps, Epi epi) {
    __shared__ float red[G > 1 ? 2 : 1][4 * ROWS];
    __shared__ float nred[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t nbase = (int64_t)blockIdx.x * G * ROWS;
    const int64_t k0 = (int64_t)tid * kRec;
    auto prow = [&](int g, int r) -> int64_t {  // plane row of logical row nbase + g ROWS + r (clamped)
        const int64_t n = nbase + (int64_t)g * ROWS + r;
        return n < N ? n : N - 1;
    };
    u32x4 xr[NS][2], nr[NS][2];
    bool live[NS];
    QRec<T> er[NS];
    const bool embed = src.emb.nib != nullptr;
    const int64_t trow = embed ? src.token->token : 0;
#pragma unroll
    for (int i = 0; i < NS; i++) {
        const int64_t k = k0 + (int64_t)i * kQfSlab;
        live[i] = k < K;
        const int64_t kc = live[i] ? k : 0;
        if (embed) {
            er[i] = qf_load<T>(src.emb, trow, kc / kRec, K);
        } else {
            xr[i][0] = ld16(src.x + kc);
            xr[i][1] = ld16(src.x + kc + 8);
        }
        if (NORM) {
            nr[i][0] = ld16(nw + kc);
            nr[i][1] = ld16(nw + kc + 8);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    const int64_t kf = k0 < K ? k0 : 0;
    constexpr int TT = G * NS, D = TT < kGemvDepth ? TT : kGemvDepth;
    QRec<T> qb[D][ROWS];
    auto request = [&](int st) {
        const int g = st / NS, i = st % NS;
        const int64_t k = k0 + (int64_t)i * kQfSlab;
        const int64_t kc = k < K ? k : kf;  // dead lanes of a partial slab re-read their first record
#pragma unroll
        for (int r = 0; r < ROWS; r++) qb[st % D][r] = qf_load<T>(w, prow(g, r), kc / kRec, K);
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
        if (embed) qf_deq16<T>(er[i], xr[i]);
#pragma unroll
        for (int c = 0; c < 2; c++) {
            if (!live[i]) xr[i][c] = u32x4{0u, 0u, 0u, 0u};
            if (xcopy && live[i]) st16(xcopy + k0 + (int64_t)i * kQfSlab + 8 * c, xr[i][c]);
            if (NORM) ss = sumsq8(xr[i][c], ss);
        }
    }
    if (NORM) {
        ss = block_sum<kThreads / kWave, false>(ss, nred);
        const h16 inv = (h16)(1.0f / sqrtf(ss / (float)K + eps));
#pragma unroll
        for (int i = 0; i < NS; i++)
#pragma unroll
            for (int c = 0; c < 2; c++) xr[i][c] = norm8(xr[i][c], nr[i][c], inv);
    }
    unsigned xp[NS][8];
    float xs[NS];
#pragma unroll
    for (int i = 0; i < NS; i++) {
        qf_perm_x(xr[i], xp[i]);
        xs[i] = 0.0f;
        if constexpr (T == AESIR_GGML_Q4_K) {
            const h16x2 one = {(h16)1.0f, (h16)1.0f};
#pragma unroll
            for (int f = 0; f < 8; f++) xs[i] = __builtin_amdgcn_fdot2(as_h2(xp[i][f]), one, xs[i], false);
        }
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
            for (int r = 0; r < ROWS; r++) acc[r] = qf_dot<T>(qb[st % D][r], xp[i], xs[i], acc[r]);
            if (st + D < TT) {
                request(st + D);
                const int gn = (st + D) / NS;
                if ((st + D) % NS == 0) pre[gn] = epi.template prefetch<ROWS>(nbase + (int64_t)gn * ROWS, 0, N, tid);
            }
        }
        wave_multi_sum<ROWS>(acc, lane);
        constexpr int GW = kWave / ROWS;
        float *rg = red[g & (G > 1 ? 1 : 0)];
        if ((lane & (GW - 1)) == 0) rg[wave * ROWS + lane / GW] = acc[0];
        __syncthreads();
        epi.template apply<ROWS>(nbase + (int64_t)g * ROWS, 0, N, RowSums<ROWS>{rg}, tid, pre[g]);
    }
}

template <int T, int ROWS, int G, bool NORM, class Epi>
static int32_t gemv_qf_launch_t(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const QFXSrc &src, const void *nw,
                                float eps, const Epi &epi, int64_t ns, const dim3 &grid) {
    switch (ns) {
#define AESIR_QF_NS(NSV)                                                                                         \
    case NSV:                                                                                                   \
        hipLaunchKernelGGL((gemv_qf_kernel<T, ROWS, NSV, G, NORM, Epi>), grid, dim3(kThreads), 0, s, w, N, K, src, \
                           (const h16 *)nw, eps, epi);                                                          \
        return AESIR_OK;
        AESIR_QF_NS(1)
        AESIR_QF_NS(2)
        AESIR_QF_NS(3)
        AESIR_QF_NS(4)
        AESIR_QF_NS(5)
        AESIR_QF_NS(6)
        AESIR_QF_NS(7)
#undef AESIR_QF_NS
        default: return fail(AESIR_ERR_UNSUPPORTED, "quantized GEMV: K = %lld exceeds %lld", (long long)K,
                             (long long)(kQfSlab * kQfMaxSlabs));
    }
}

template <int ROWS, int G, bool NORM, class Epi>
static int32_t gemv_qf_dispatch(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const QFXSrc &src, const void *nw,
                                float eps, const Epi &epi, const char *name) {
    AESIR_TRY(qf_check(w.type, K, name));
    if (src.emb.nib && src.emb.type != w.type) return fail(AESIR_ERR_INVALID, "%s: embedding type differs", name);
    const void *xp = src.emb.nib ? (const void *)src.emb.nib : (const void *)src.x;
    if (((uintptr_t)w.nib & 7) || ((uintptr_t)xp & 15) || (NORM && ((uintptr_t)nw & 15)) ||
        (src.xcopy && ((uintptr_t)src.xcopy & 15)))
        return fail(AESIR_ERR_UNSUPPORTED, "%s: quantized GEMV needs aligned operands", name);
    const dim3 grid((unsigned)((N + ROWS * G - 1) / (ROWS * G)));
    if (grid.x == 0) return AESIR_OK;
    const int64_t ns = (K + kQfSlab - 1) / kQfSlab;
    int32_t rc;
    if (w.type == AESIR_GGML_Q4_0)
        rc = gemv_qf_launch_t<AESIR_GGML_Q4_0, ROWS, G, NORM, Epi>(s, w, N, K, src, nw, eps, epi, ns, grid);
    else if (w.type == AESIR_GGML_Q4_K)
        rc = gemv_qf_launch_t<AESIR_GGML_Q4_K, ROWS, G, NORM, Epi>(s, w, N, K, src, nw, eps, epi, ns, grid);
    else
        rc = gemv_qf_launch_t<AESIR_GGML_Q6_K, ROWS, G, NORM, Epi>(s, w, N, K, src, nw, eps, epi, ns, grid);
    AESIR_TRY(rc);
    AESIR_LAUNCH_CHECK(name);
    return AESIR_OK;
}

int32_t launch_qf_gemv_store(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const void *x, void *y) {
    EpiStore e{(h16 *)y, N};
    return gemv_qf_dispatch<kQfRows, 1, false>(s, w, N, K, QFXSrc{(const h16 *)x, QFMat{}, nullptr, nullptr}, nullptr,
                                               0.0f, e, "gemv_qf_store");
}

int32_t launch_qf_gemv_residual(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const void *x_in, void *x) {
    EpiResidual e{(h16 *)x};
    return gemv_qf_dispatch<kQfRows, 1, false>(s, w, N, K, QFXSrc{(const h16 *)x_in, QFMat{}, nullptr, nullptr},
                                               nullptr, 0.0f, e, "gemv_qf_residual");
}

int32_t launch_qf_gate_up_swiglu(hipStream_t s, const void *x, const void *norm_w, float eps, const QFMat &w,
                                 int64_t ffn, int64_t dim, void *act) {
    EpiSwiglu e{(h16 *)act};
    return gemv_qf_dispatch<kQfRows, 2, true>(s, w, 2 * ffn, dim, QFXSrc{(const h16 *)x, QFMat{}, nullptr, nullptr},
                                              norm_w, eps, e, "gemv_qf_gate_up");
}

int32_t launch_qf_qkv_rope_kv(hipStream_t s, const QkvArgs &a, const EpiQkv &e) {
    const QFXSrc src = a.eq.nib ? QFXSrc{nullptr, a.eq, a.state, (h16 *)a.x}
                                : QFXSrc{(const h16 *)a.x, QFMat{}, nullptr, nullptr};
    return gemv_qf_dispatch<kQfRows, 1, true>(s, a.wq, a.dim + 2 * a.kvd, a.dim, src, a.norm_w, a.eps, e,
                                              "gemv_qf_qkv_rope_kv");
}

int32_t launch_qf_lm_head(hipStream_t s, const LmHeadArgs &a, const EpiLmHead &e) {
    return gemv_qf_dispatch<8, 1, true>(s, a.wq, a.vocab, a.dim, QFXSrc{(const h16 *)a.x, QFMat{}, nullptr, nullptr},
                                        a.norm_w, a.eps, e, "gemv_qf_lm_head");
}

}  // namespace aesir
