// 4-bit and K-quant weights on gfx950: GGML Q4_0 (with the reference's gemm_q4_0 rounding,
// core/compute.mojo:876-912) and GGML's Q4_K / Q6_K super-blocks.
//
// GGUF stores these as packed blocks of 18, 144 and 210 bytes whose nibble order suits a CPU
// loop, not a wave: the bytes of one block are read by one lane, and 210 is not even 4-byte
// aligned. At upload every matrix is repacked (QFMat in kernels.hpp) into records of 16 weights:
// 8 nibble bytes per record, byte j holding weights j and 8 + j, so that masking a record word
// with 0x000F000F or 0x00F000F0 and OR-ing 0x64006400 yields the f16 pair (1024 + q_a, 1024 +
// q_b) or (1024 + 16 q_a, 1024 + 16 q_b) for weights (a, a + 2); plus small planes of per-block
// scales and, for Q6_K, one word of high bits per record. A decode GEMV lane multiplies one
// 32-weight chunk (two records, one 16-byte load) per row and slab, with x held in registers in
// the matching pair order.
//
// Arithmetic per type:
//   Q4_0  w = f16(f16(q - 8) * d), the reference's dequantize_q4_0 (compute.mojo:266-280): the
//         pair q - 8 is exact in f16, the packed f16 multiply by d rounds once; then f32
//         v_dot2_f32_f16 accumulation as in the F16 path.
//   Q4_K  w = (d * sc) * q - dmin * m, GGML's value in f32. Per 32-weight sub-block: S = sum x q
//         with q exact in f16, X = sum x; contribution (d sc) S - (dmin m) X in f32.
//   Q6_K  w = (d * sc) * (q - 32): per record S = sum x (q - 32) with the 6-bit value exact in
//         f16, contribution (d sc) S in f32.
// The K-quant dot products therefore use the f32 weights GGML defines, not f16-rounded ones.
#include <atomic>
#include <type_traits>

#include "device.hpp"
#include "gemv_common.hpp"
#include "kernels.hpp"

namespace aesir {

constexpr int kRec = 16;                  // weights per record
constexpr unsigned kMagic = 0x64006400u;  // f16 1024 in both halves
// Decode GEMV shape: rows per group (the epilogue's unit), groups per workgroup (the gate/up
// projection runs two), weight requests in flight per lane (in (group, slab) steps), and the
// most slabs instantiated for 1, 2 and 4 sub-groups (K <= 32768, 8192, 6144).
constexpr int kQfGroupRows = 8;
constexpr int kQfGroups = 1;
constexpr int kQfGroupsFfn = 2;
constexpr int kQfDepth = 2;
constexpr int kQfMaxSlabs[3] = {4, 2, 3};


bool qf_type(int32_t t) { return t == AESIR_GGML_Q4_0 || t == AESIR_GGML_Q4_K || t == AESIR_GGML_Q6_K; }

// Nibble pair f of a record holds weights a and a + 2, a = {0, 1, 4, 5, 8, 9, 12, 13}[f]: pairs
// 0-3 are low nibbles, 4-7 high nibbles. In the Q6_K high-bit word, pair f's two 2-bit fields sit
// 16 bits apart at qf_hb_off(f) = {0, 2, 8, 10}[f & 3] + 4 (f >> 2) and 16 above, so that one
// shift by 4 - {0, 2, 8, 10}[f & 3] serves a low pair (fields to bits 4, 20, above its nibbles)
// and a high pair (to bits 8, 24, above its 16-scaled nibbles).
__host__ __device__ __forceinline__ int qf_hb_off(int f) { return ((f & 1) << 1) + ((f & 2) << 2) + ((f >> 2) << 2); }
// Bit position of the high 2 bits of record weight i.
__host__ __device__ __forceinline__ int qf_hb_pos(int i) {
    const int a = i & ~2, f = (a & 1) | (((a >> 2) & 1) << 1) | (((a >> 3) & 1) << 2);
    return qf_hb_off(f) + 16 * ((i >> 1) & 1);
}

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
    const int s = 4 - qf_hb_off(f);
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

// A lane of the decode GEMV owns one 32-weight chunk of a row per slab: two records, i.e. one
// 16-byte nibble load (c = chunk index, k = 32 c). Q4_0 chunks are GGML blocks and Q4_K chunks
// are sub-blocks, so each needs one scale entry per row.
constexpr int kChunk = 32;

// Register-held constants: the and-or and packed-f16 forms below take a mask or bias from a
// register (one VOP3 instruction holds at most one literal), which the compiler does not arrange
// by itself; without them every nibble pair costs a shift, an AND and an OR.
__device__ __forceinline__ unsigned sreg(unsigned v) {
    unsigned r;
    asm("s_mov_b32 %0, %1" : "=s"(r) : "i"(v));
    return r;
}
__device__ __forceinline__ unsigned vreg(unsigned v) {
    unsigned r;
    asm("v_mov_b32 %0, %1" : "=v"(r) : "i"(v));
    return r;
}

struct QfRegs {
    unsigned lo, hi, magic;  // nibble masks 0x000F000F / 0x00F000F0, f16 1024 in both halves
    unsigned hlo, hhi;       // Q6_K high-bit masks 0x00300030 / 0x03000300
    __device__ __forceinline__ static QfRegs make() {
        return QfRegs{sreg(0x000F000Fu), sreg(0x00F000F0u), vreg(kMagic), sreg(0x00300030u), sreg(0x03000300u)};
    }
};

// One row's chunk as loaded.
template <int T>
struct QChunk;
template <>
struct QChunk<AESIR_GGML_Q4_0> {
    u32x4 nib;
    unsigned d;  // f16 scale in the low half
};
template <>
struct QChunk<AESIR_GGML_Q4_K> {
    u32x4 nib;
    unsigned scm;  // scale | min << 8
    unsigned dd;   // f16 d | f16 dmin << 16
};
template <>
struct QChunk<AESIR_GGML_Q6_K> {
    u32x4 nib;
    u32x2 hb;      // high-bit words of the two records
    unsigned sc2;  // int8 scales of the two records
    unsigned d;    // f16 super-block scale in the low half
};

// Buffer resources of a matrix's planes (range-checked loads with the row offset in an SGPR).
struct QfRsrc {
    __amdgpu_buffer_rsrc_t nib, hb, s0, s1;
    int nb, hbb, s0b, s1b;  // bytes per row of each plane
};

__device__ __forceinline__ QfRsrc qf_rsrc(const QFMat &w, int32_t type, int64_t N, int64_t K) {
    QfRsrc r;
    r.nb = (int)qf_plane_row_bytes(type, 0, K);
    r.hbb = type == AESIR_GGML_Q6_K ? (int)qf_plane_row_bytes(type, 1, K) : 0;
    r.s0b = (int)qf_plane_row_bytes(type, 2, K);
    r.s1b = type == AESIR_GGML_Q4_0 ? 0 : (int)qf_plane_row_bytes(type, 3, K);
    r.nib = __builtin_amdgcn_make_buffer_rsrc((void *)w.nib, 0, (int)(N * r.nb), 0x00020000);
    r.hb = __builtin_amdgcn_make_buffer_rsrc((void *)w.hb, 0, (int)(N * r.hbb), 0x00020000);
    r.s0 = __builtin_amdgcn_make_buffer_rsrc((void *)w.s0, 0, (int)(N * r.s0b), 0x00020000);
    r.s1 = __builtin_amdgcn_make_buffer_rsrc((void *)w.s1, 0, (int)(N * r.s1b), 0x00020000);
    return r;
}

// Chunk c of plane row n (n wave-uniform: the row offsets go in SGPRs).
template <int T>
__device__ __forceinline__ QChunk<T> qf_chunk_load(const QfRsrc &r, int n, int c) {
    QChunk<T> q;
    q.nib = __builtin_amdgcn_raw_buffer_load_b128(r.nib, c * 16, n * r.nb, 2);
    if constexpr (T == AESIR_GGML_Q4_0) {
        q.d = __builtin_amdgcn_raw_buffer_load_b16(r.s0, c * 2, n * r.s0b, 0);
    } else if constexpr (T == AESIR_GGML_Q4_K) {
        q.scm = __builtin_amdgcn_raw_buffer_load_b16(r.s0, c * 2, n * r.s0b, 0);
        q.dd = __builtin_amdgcn_raw_buffer_load_b32(r.s1, (c >> 3) * 4, n * r.s1b, 0);
    } else {
        q.hb = __builtin_amdgcn_raw_buffer_load_b64(r.hb, c * 8, n * r.hbb, 2);
        q.sc2 = __builtin_amdgcn_raw_buffer_load_b16(r.s0, c * 2, n * r.s0b, 0);
        q.d = __builtin_amdgcn_raw_buffer_load_b16(r.s1, (c >> 3) * 2, n * r.s1b, 0);
    }
    return q;
}

// acc + this chunk's share of the row's dot product. xp: the chunk's x in pair order (record j
// pair f at xp[8 j + f]); X: sum of the chunk's 32 x values (Q4_K).
//
// Nibble pairs come out of a word v of record bytes as (v & 0x000F000F) | magic = 1024 + q for
// the low nibbles of bytes 0 and 2 and (v & 0x00F000F0) | magic = 1024 + 16 q for the high ones;
// v >> 8 gives bytes 1 and 3. Word 0 of a record yields pairs f = 0, 1 (low) and 4, 5 (high),
// word 1 pairs 2, 3 and 6, 7. All values are exact in f16: Q4_0 turns them into q - 8 (adding
// -1032, or times 1/16 plus -72), Q4_K/Q6_K keep separate sums for the 16-scaled pairs and scale
// by 1/16 in f32.
template <int T>
__device__ __forceinline__ float qf_chunk_dot(const QChunk<T> &q, const unsigned (&xp)[16], float X, float acc,
                                              const QfRegs &k) {
    const unsigned nw[4] = {q.nib.x, q.nib.y, q.nib.z, q.nib.w};
    if constexpr (T == AESIR_GGML_Q4_0) {
        const h16 d = bits_to_h((uint16_t)(q.d & 0xffffu));
        const h16x2 dd = {d, d};
        const h16x2 blo = {(h16)-1032.0f, (h16)-1032.0f}, s16 = {(h16)0.0625f, (h16)0.0625f},
                    bhi = {(h16)-72.0f, (h16)-72.0f};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const unsigned v = nw[j], t = v >> 8;
            const unsigned *x = xp + 8 * (j >> 1) + 2 * (j & 1);
            acc = __builtin_amdgcn_fdot2((as_h2((v & k.lo) | k.magic) + blo) * dd, as_h2(x[0]), acc, false);
            acc = __builtin_amdgcn_fdot2((as_h2((t & k.lo) | k.magic) + blo) * dd, as_h2(x[1]), acc, false);
            acc = __builtin_amdgcn_fdot2(__builtin_elementwise_fma(as_h2((v & k.hi) | k.magic), s16, bhi) * dd,
                                         as_h2(x[4]), acc, false);
            acc = __builtin_amdgcn_fdot2(__builtin_elementwise_fma(as_h2((t & k.hi) | k.magic), s16, bhi) * dd,
                                         as_h2(x[5]), acc, false);
        }
        return acc;
    } else if constexpr (T == AESIR_GGML_Q4_K) {
        const h16x2 b = {(h16)-1024.0f, (h16)-1024.0f};
        float slo = 0.0f, shi = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const unsigned v = nw[j], t = v >> 8;
            const unsigned *x = xp + 8 * (j >> 1) + 2 * (j & 1);
            slo = __builtin_amdgcn_fdot2(as_h2((v & k.lo) | k.magic) + b, as_h2(x[0]), slo, false);
            slo = __builtin_amdgcn_fdot2(as_h2((t & k.lo) | k.magic) + b, as_h2(x[1]), slo, false);
            shi = __builtin_amdgcn_fdot2(as_h2((v & k.hi) | k.magic) + b, as_h2(x[4]), shi, false);
            shi = __builtin_amdgcn_fdot2(as_h2((t & k.hi) | k.magic) + b, as_h2(x[5]), shi, false);
        }
        const float S = fmaf(shi, 0.0625f, slo);
        const float d = (float)bits_to_h((uint16_t)(q.dd & 0xffffu)), dm = (float)bits_to_h((uint16_t)(q.dd >> 16));
        const float a = d * (float)(q.scm & 0xffu), bb = dm * (float)((q.scm >> 8) & 0xffu);
        return acc + (a * S - bb * X);
    } else {
        // High bits: record word h holds pair f's two 2-bit fields at o + 4 (f >> 2) and 16 above,
        // o = {0, 2, 8, 10}[f & 3]; h shifted by 4 - o puts the low pairs' fields at bits 4 and
        // 20 and the high pairs' at bits 8 and 24, next to their nibbles.
        const h16x2 blo = {(h16)-1056.0f, (h16)-1056.0f}, bhi = {(h16)-1536.0f, (h16)-1536.0f};
        const float d = (float)bits_to_h((uint16_t)(q.d & 0xffffu));
        const unsigned hw[2] = {q.hb.x, q.hb.y};
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const unsigned h = hw[r];
            const unsigned hs[4] = {h << 4, h << 2, h >> 4, h >> 6};
            float slo = 0.0f, shi = 0.0f;
#pragma unroll
            for (int w = 0; w < 2; w++) {
                const unsigned v = nw[2 * r + w], t = v >> 8;
                const unsigned ha = hs[2 * w], hb = hs[2 * w + 1];
                const unsigned *x = xp + 8 * r + 2 * w;
                slo = __builtin_amdgcn_fdot2(as_h2((ha & k.hlo) | ((v & k.lo) | k.magic)) + blo, as_h2(x[0]), slo, false);
                slo = __builtin_amdgcn_fdot2(as_h2((hb & k.hlo) | ((t & k.lo) | k.magic)) + blo, as_h2(x[1]), slo, false);
                shi = __builtin_amdgcn_fdot2(as_h2((ha & k.hhi) | ((v & k.hi) | k.magic)) + bhi, as_h2(x[4]), shi, false);
                shi = __builtin_amdgcn_fdot2(as_h2((hb & k.hhi) | ((t & k.hi) | k.magic)) + bhi, as_h2(x[5]), shi, false);
            }
            const float sc = (float)(int8_t)((q.sc2 >> (8 * r)) & 0xffu);
            acc += (d * sc) * fmaf(shi, 0.0625f, slo);
        }
        return acc;
    }
}

// Row sums of a workgroup group of RT rows reduced by P waves each: red[w * RT + r].
template <int RT, int P>
struct QfRowSums {
    const float *red;
    __device__ __forceinline__ float operator[](int r) const {
        if constexpr (P == 4) return (red[r] + red[RT + r]) + (red[2 * RT + r] + red[3 * RT + r]);
        if constexpr (P == 2) return red[r] + red[RT + r];
        return red[r];
    }
};

// x source: x itself, or (layer 0) row token->token of the repacked embedding table, dequantized
// in registers, with workgroup 0 writing the row to xcopy (the residual stream).
struct QFXSrc {
    const h16 *x;
    QFMat emb;
    const DecodeState *token;
    h16 *xcopy;
};

// The 256 threads form H sub-groups of LPR = 256 / H lanes; sub-group h multiplies rows
// h ROWS .. h ROWS + ROWS - 1 of each RT = H ROWS-row group, lane p taking chunk p + LPR i of
// slab i (NS slabs cover K). A workgroup runs G groups. x stays in registers (RMS-normalized once,
// then put in pair order); the chunk requests run D (group, slab) steps ahead through a register
// ring; each group ends in a wave reduction, one LDS exchange and the fused epilogue.
template <int T, int ROWS, int H, int NS, int G, bool NORM, class Epi>
__global__ __launch_bounds__(kThreads) void gemv_qf_kernel(QFMat w, int64_t N, int64_t K, QFXSrc src,
                                                           const h16 *__restrict__ nw, float eps, Epi epi) {
    constexpr int LPR = kThreads / H, WPS = LPR / kWave, RT = H * ROWS;
    __shared__ float red[G > 1 ? 2 : 1][WPS * RT];
    __shared__ float nred[4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = wave / WPS, p = tid % LPR;
    const int64_t nbase = (int64_t)blockIdx.x * G * RT;
    const int chunks = (int)(K / kChunk);
    const QfRsrc rs = qf_rsrc(w, T, N, K);
    auto row = [&](int g, int r) -> int {  // plane row of row r of sub-group h in group g (clamped)
        const int64_t n = nbase + (int64_t)g * RT + h * ROWS + r;
        return (int)(n < N ? n : N - 1);
    };
    u32x4 xr[NS][4], nr[NS][4];
    bool live[NS];
    const bool embed = src.emb.nib != nullptr;
    const int64_t trow = embed ? src.token->token : 0;
#pragma unroll
    for (int i = 0; i < NS; i++) {
        const int c = p + LPR * i;
        live[i] = c < chunks;
        const int64_t k = live[i] ? (int64_t)c * kChunk : 0;
        if (embed) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                u32x4 o[2];
                qf_deq16<T>(qf_load<T>(src.emb, trow, k / kRec + j, K), o);
                xr[i][2 * j] = o[0];
                xr[i][2 * j + 1] = o[1];
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) xr[i][q] = ld16(src.x + k + 8 * q);
        }
        if (NORM)
#pragma unroll
            for (int q = 0; q < 4; q++) nr[i][q] = ld16(nw + k + 8 * q);
    }
    __builtin_amdgcn_sched_barrier(0);
    constexpr int TT = G * NS, D = TT < kQfDepth ? TT : kQfDepth;
    QChunk<T> qb[D][ROWS];
    auto request = [&](int st) {
        const int g = st / NS, i = st % NS;
        const int c = p + LPR * i;
        const int cc = c < chunks ? c : 0;  // dead lanes of a partial slab re-read chunk 0
#pragma unroll
        for (int r = 0; r < ROWS; r++) qb[st % D][r] = qf_chunk_load<T>(rs, row(g, r), cc);
    };
#pragma unroll
    for (int st = 0; st < D; st++) request(st);
    __builtin_amdgcn_sched_barrier(0);
    using Pre = decltype(epi.template prefetch<RT>(0, 0, N, tid));
    Pre pre[G];
#pragma unroll
    for (int g = 0; g < G; g++)
        if (g * NS < D) pre[g] = epi.template prefetch<RT>(nbase + (int64_t)g * RT, 0, N, tid);

    float ss = 0.0f;
    const bool first = h == 0;  // sub-group 0 holds one copy of x
    h16 *xcopy = (src.xcopy && blockIdx.x == 0 && first) ? src.xcopy : nullptr;
#pragma unroll
    for (int i = 0; i < NS; i++) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (!live[i]) xr[i][q] = u32x4{0u, 0u, 0u, 0u};
            if (xcopy && live[i]) st16(xcopy + (int64_t)(p + LPR * i) * kChunk + 8 * q, xr[i][q]);
            if (NORM && first) ss = sumsq8(xr[i][q], ss);
        }
    }
    if (NORM) {
        ss = block_sum<kThreads / kWave, false>(ss, nred);
        const h16 inv = (h16)(1.0f / sqrtf(ss / (float)K + eps));
#pragma unroll
        for (int i = 0; i < NS; i++)
#pragma unroll
            for (int q = 0; q < 4; q++) xr[i][q] = norm8(xr[i][q], nr[i][q], inv);
    }
    unsigned xp[NS][16];
    float X[NS];
#pragma unroll
    for (int i = 0; i < NS; i++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            unsigned part[8];
            const u32x4 pr[2] = {xr[i][2 * j], xr[i][2 * j + 1]};
            qf_perm_x(pr, part);
#pragma unroll
            for (int f = 0; f < 8; f++) xp[i][8 * j + f] = part[f];
        }
        X[i] = 0.0f;
        if constexpr (T == AESIR_GGML_Q4_K) {
            const h16x2 one = {(h16)1.0f, (h16)1.0f};
#pragma unroll
            for (int f = 0; f < 16; f++) X[i] = __builtin_amdgcn_fdot2(as_h2(xp[i][f]), one, X[i], false);
        }
    }
    const QfRegs kr = QfRegs::make();
#pragma unroll
    for (int g = 0; g < G; g++) {
        float acc[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; r++) acc[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const int st = g * NS + i;
#pragma unroll
            for (int r = 0; r < ROWS; r++) acc[r] = qf_chunk_dot<T>(qb[st % D][r], xp[i], X[i], acc[r], kr);
            if (st + D < TT) {
                request(st + D);
                const int gn = (st + D) / NS;
                if ((st + D) % NS == 0) pre[gn] = epi.template prefetch<RT>(nbase + (int64_t)gn * RT, 0, N, tid);
            }
        }
        wave_multi_sum<ROWS>(acc, lane);
        constexpr int GW = kWave / ROWS;
        float *rg = red[g & (G > 1 ? 1 : 0)];
        if ((lane & (GW - 1)) == 0) rg[(wave % WPS) * RT + h * ROWS + lane / GW] = acc[0];
        __syncthreads();
        epi.template apply<RT>(nbase + (int64_t)g * RT, 0, N, QfRowSums<RT, WPS>{rg}, tid, pre[g]);
    }
}

// Sub-group count for a row length: the fewest lanes left idle by the last slab, then the fewer
// slabs. Returns 0 when no instantiated shape covers K.
static int qf_pick_h(int64_t K) {
    int best = 0;
    int64_t best_waste = INT64_MAX, best_ns = 0;
    for (int h : {1, 2, 4}) {
        const int64_t slab = (int64_t)(kThreads / h) * kChunk, ns = (K + slab - 1) / slab;
        if (ns > kQfMaxSlabs[h == 1 ? 0 : h == 2 ? 1 : 2]) continue;
        const int64_t waste = ns * slab - K;
        if (waste < best_waste || (waste == best_waste && ns < best_ns)) {
            best = h;
            best_waste = waste;
            best_ns = ns;
        }
    }
    return best;
}

template <int T, int ROWS, int H, int G, bool NORM, class Epi>
static int32_t gemv_qf_launch_h(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const QFXSrc &src, const void *nw,
                                float eps, const Epi &epi, int64_t ns) {
    const dim3 grid((unsigned)((N + (int64_t)H * ROWS * G - 1) / ((int64_t)H * ROWS * G)));
    switch (ns) {
#define AESIR_QF_NS(NSV)                                                                                          \
    case NSV:                                                                                                    \
        if constexpr (NSV <= kQfMaxSlabs[H == 1 ? 0 : H == 2 ? 1 : 2]) {                                        \
            hipLaunchKernelGGL((gemv_qf_kernel<T, ROWS, H, NSV, G, NORM, Epi>), grid, dim3(kThreads), 0, s, w, N, K, \
                               src, (const h16 *)nw, eps, epi);                                                  \
            return AESIR_OK;                                                                                     \
        }                                                                                                        \
        break;
        AESIR_QF_NS(1)
        AESIR_QF_NS(2)
        AESIR_QF_NS(3)
        AESIR_QF_NS(4)
#undef AESIR_QF_NS
        default: break;
    }
    return fail(AESIR_ERR_UNSUPPORTED, "quantized GEMV: K = %lld exceeds %lld", (long long)K,
                (long long)(kThreads * kChunk * kQfMaxSlabs[0]));
}

// RT: rows per group of the workgroup, split over the H sub-groups.
template <int RT, int G, bool NORM, class Epi, int T>
static int32_t gemv_qf_launch_t(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const QFXSrc &src, const void *nw,
                                float eps, const Epi &epi) {
    const int h = qf_pick_h(K);
    if (h == 0)
        return fail(AESIR_ERR_UNSUPPORTED, "quantized GEMV: K = %lld exceeds %lld", (long long)K,
                    (long long)(kThreads * kChunk * kQfMaxSlabs[0]));
    const int64_t slab = (int64_t)(kThreads / h) * kChunk, ns = (K + slab - 1) / slab;
    // one sub-group: half the rows per group (register budget of the long-K slabs), except for the
    // lm_head, whose argmax partials are per RT rows
    constexpr int R1 = std::is_same<Epi, EpiLmHead>::value ? RT : RT / 2;
    if (h == 1) return gemv_qf_launch_h<T, R1, 1, G, NORM, Epi>(s, w, N, K, src, nw, eps, epi, ns);
    if (h == 2) return gemv_qf_launch_h<T, RT / 2, 2, G, NORM, Epi>(s, w, N, K, src, nw, eps, epi, ns);
    return gemv_qf_launch_h<T, RT / 4, 4, G, NORM, Epi>(s, w, N, K, src, nw, eps, epi, ns);
}

template <int RT, int G, bool NORM, class Epi>
static int32_t gemv_qf_dispatch(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const QFXSrc &src, const void *nw,
                                float eps, const Epi &epi, const char *name) {
    static_assert(RT % 4 == 0, "groups split over up to four sub-groups");
    AESIR_TRY(qf_check(w.type, K, name));
    if (src.emb.nib && src.emb.type != w.type) return fail(AESIR_ERR_INVALID, "%s: embedding type differs", name);
    const void *xp = src.emb.nib ? (const void *)src.emb.nib : (const void *)src.x;
    if (((uintptr_t)w.nib & 15) || ((uintptr_t)xp & 15) || (NORM && ((uintptr_t)nw & 15)) ||
        (src.xcopy && ((uintptr_t)src.xcopy & 15)))
        return fail(AESIR_ERR_UNSUPPORTED, "%s: quantized GEMV needs 16-byte aligned operands", name);
    // plane offsets are 32-bit in the buffer loads
    if (N <= 0) return AESIR_OK;
    if (mul_checked(N, qf_plane_row_bytes(w.type, 0, K)) > INT32_MAX)
        return fail(AESIR_ERR_UNSUPPORTED, "%s: matrix of %lld x %lld exceeds 2 GiB of 4-bit weights", name, (long long)N,
                    (long long)K);
    int32_t rc;
    if (w.type == AESIR_GGML_Q4_0)
        rc = gemv_qf_launch_t<RT, G, NORM, Epi, AESIR_GGML_Q4_0>(s, w, N, K, src, nw, eps, epi);
    else if (w.type == AESIR_GGML_Q4_K)
        rc = gemv_qf_launch_t<RT, G, NORM, Epi, AESIR_GGML_Q4_K>(s, w, N, K, src, nw, eps, epi);
    else
        rc = gemv_qf_launch_t<RT, G, NORM, Epi, AESIR_GGML_Q6_K>(s, w, N, K, src, nw, eps, epi);
    AESIR_TRY(rc);
    AESIR_LAUNCH_CHECK(name);
    return AESIR_OK;
}

int32_t launch_qf_gemv_store(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const void *x, void *y) {
    EpiStore e{(h16 *)y, N};
    return gemv_qf_dispatch<kQfGroupRows, kQfGroups, false>(s, w, N, K, QFXSrc{(const h16 *)x, QFMat{}, nullptr, nullptr},
                                                          nullptr, 0.0f, e, "gemv_qf_store");
}

int32_t launch_qf_gemv_residual(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const void *x_in, void *x) {
    EpiResidual e{(h16 *)x};
    return gemv_qf_dispatch<kQfGroupRows, kQfGroups, false>(s, w, N, K, QFXSrc{(const h16 *)x_in, QFMat{}, nullptr, nullptr},
                                                          nullptr, 0.0f, e, "gemv_qf_residual");
}

int32_t launch_qf_gate_up_swiglu(hipStream_t s, const void *x, const void *norm_w, float eps, const QFMat &w,
                                 int64_t ffn, int64_t dim, void *act) {
    EpiSwiglu e{(h16 *)act};
    return gemv_qf_dispatch<kQfGroupRows, kQfGroupsFfn, true>(s, w, 2 * ffn, dim,
                                                            QFXSrc{(const h16 *)x, QFMat{}, nullptr, nullptr}, norm_w,
                                                            eps, e, "gemv_qf_gate_up");
}

int32_t launch_qf_qkv_rope_kv(hipStream_t s, const QkvArgs &a, const EpiQkv &e) {
    const QFXSrc src = a.eq.nib ? QFXSrc{nullptr, a.eq, a.state, (h16 *)a.x}
                                : QFXSrc{(const h16 *)a.x, QFMat{}, nullptr, nullptr};
    return gemv_qf_dispatch<kQfGroupRows, kQfGroups, true>(s, a.wq, a.dim + 2 * a.kvd, a.dim, src, a.norm_w, a.eps, e,
                                                         "gemv_qf_qkv_rope_kv");
}

// 8 rows per group: one argmax partial per 8 logits (lm_head_groups).
int32_t launch_qf_lm_head(hipStream_t s, const LmHeadArgs &a, const EpiLmHead &e) {
    return gemv_qf_dispatch<8, 1, true>(s, a.wq, a.vocab, a.dim, QFXSrc{(const h16 *)a.x, QFMat{}, nullptr, nullptr},
                                        a.norm_w, a.eps, e, "gemv_qf_lm_head");
}

}  // namespace aesir
