// 2- to 6-bit weights on gfx950: GGML Q4_0, Q4_1, Q5_0 and Q5_1 (with the reference's
// gemm_q4_0 / _q4_1 / _q5_0 / _q5_1 rounding, core/compute.mojo:876-1036) and GGML's Q2_K / Q3_K /
// Q4_K / Q5_K / Q6_K super-blocks. Q2_K and Q3_K keep GGUF's bit width: the low 2 bits of each
// weight as crumbs (4 bytes per record) and, for Q3_K, the third bits in a word per record pair,
// next to the crumbs in the quant plane; a lane spreads them into the nibble words the 4-bit
// dequantization takes.
//
// GGUF stores these as packed blocks of 18 to 210 bytes whose nibble order suits a CPU
// loop, not a wave: the bytes of one block are read by one lane, and 210 is not even 4-byte
// aligned. At upload every matrix is repacked (QFMat in kernels.hpp) into records of 16 weights:
// 8 nibble bytes per record, byte j holding weights j and 8 + j, so that masking a record word
// with 0x000F000F or 0x00F000F0 and OR-ing 0x64006400 yields the f16 pair (1024 + q_a, 1024 +
// q_b) or (1024 + 16 q_a, 1024 + 16 q_b) for weights (a, a + 2); plus small planes of per-block
// scales and, for Q6_K, one word of high bits per record (for the 5-bit types, one word of fifth
// bits per record pair). The planes are tiled in 16-row x
// 128-weight tiles, so that lane l of a wave reading 16 bytes at 16 l gets two records of row
// l % 16: the A operand of v_mfma_f32_16x16x32_f16 for four matrix-core steps once dequantized.
// The decode GEMV dequantizes in registers and multiplies on the matrix cores.
//
// Weights (the f16 values that the GEMV, the dequantization for the prefill GEMMs and the
// read-back all produce, bit for bit):
//   Q4_0  w = f16(f16(q - 8) * d), the reference's dequantize_q4_0 (compute.mojo:266-280): q - 8
//         is exact in f16, the product rounds once.
//   Q4_K  w = f16(a q - b), one fused multiply-add in f16, with a = f16(d * sc) and
//         b = f16(dmin * m) from GGML's block fields: the f16 arithmetic of the reference's
//         dequantize_q4_k_m (compute.mojo:245-262, q * scale + min in f16).
//   Q6_K  w = f16(a (q - 32)) with a = f16(d * sc), f16 products as in the reference's
//         dequantize_q6_k_block (compute.mojo:508-527).
//   Q4_1, Q5_1  w = f16(f16(q d) + m) (dequantize_q4_1 / _q5_1, compute.mojo:282-340: the f16
//         product, then the f16 sum); Q5_0  w = f16(f16(q - 16) d) (dequantize_q5_0);
//   Q5_K  as Q4_K with the 5-bit q; Q2_K  as Q4_K with GGML's 4-bit scale and min per 16
//         weights; Q3_K  w = f16(a q) with a = f16(d * sc) and the signed 3-bit q.
// Products with x accumulate in f32 (the matrix cores, as in the F16 path's MFMA GEMMs).
#include <type_traits>

#include "device.hpp"
#include "gemv_common.hpp"
#include "kernels.hpp"
#include "mfma_gemm.hpp"

namespace aesir {

constexpr int kRec = 16;                  // weights per record
constexpr int kSeg = 128;                 // weights per tile row (8 records)
constexpr unsigned kMagic = 0x64006400u;  // f16 1024 in both halves

bool qf_type(int32_t t) {
    return t == AESIR_GGML_Q4_0 || t == AESIR_GGML_Q4_1 || t == AESIR_GGML_Q5_0 || t == AESIR_GGML_Q5_1 ||
           t == AESIR_GGML_Q2_K || t == AESIR_GGML_Q3_K || t == AESIR_GGML_Q4_K || t == AESIR_GGML_Q5_K ||
           t == AESIR_GGML_Q6_K;
}

// Type families of the repacked layout: a fifth-bit word per record pair (Q5_0, Q5_1, Q5_K); an
// f16 (d, m) pair per 32 weights (Q4_1, Q5_1); the K-quant 6-bit (scale, min) bytes with a
// super-block (d, dmin) pair (Q4_K, Q5_K).
template <int T>
constexpr bool qf_hb5() {
    return T == AESIR_GGML_Q5_0 || T == AESIR_GGML_Q5_1 || T == AESIR_GGML_Q5_K;
}
template <int T>
constexpr bool qf_dm() {
    return T == AESIR_GGML_Q4_1 || T == AESIR_GGML_Q5_1;
}
template <int T>
constexpr bool qf_kq() {
    return T == AESIR_GGML_Q4_K || T == AESIR_GGML_Q5_K;
}
template <int T>
constexpr bool qf_crumb() {
    return T == AESIR_GGML_Q2_K || T == AESIR_GGML_Q3_K;
}

// Crumb records (Q2_K, Q3_K). Nibble i of a record's crumb word holds the low 2 bits of nibble i
// of its two nibble words (bits 0-1: word 0, bits 2-3: word 1), so each word is one shift and mask
// away. The Q3_K third bits of a record pair share one word: nibble i holds them for nibble i of
// the odd record's words 0 and 1 (bits 0, 1) and the even record's (bits 2, 3); shifting the word
// left by 2 for the odd record puts its bits where the even record's are.
constexpr unsigned kCrumbMask = 0x33333333u, kThirdMask = 0x44444444u;
__host__ __device__ __forceinline__ unsigned crumb_word(unsigned w0, unsigned w1) {
    return (w0 & kCrumbMask) | ((w1 & kCrumbMask) << 2);
}
__host__ __device__ __forceinline__ unsigned third_bits(unsigned w0, unsigned w1, int odd) {
    return odd ? ((w0 & kThirdMask) >> 2) | ((w1 & kThirdMask) >> 1) : (w0 & kThirdMask) | ((w1 & kThirdMask) << 1);
}
// Nibble words of a crumb record; h: the pair's third-bit word shifted to the even record's
// positions (0 for Q2_K).
__device__ __forceinline__ u32x2 crumb_nibbles(unsigned c, unsigned h) {
    return u32x2{(c & kCrumbMask) | (h & kThirdMask), ((c >> 2) & kCrumbMask) | ((h >> 1) & kThirdMask)};
}


// Nibble pair f of a record holds weights a and a + 2, a = {0, 1, 4, 5, 8, 9, 12, 13}[f]: pairs
// 0-3 are low nibbles, 4-7 high nibbles. In the Q6_K high-bit word, pair f's two 2-bit fields sit
// 16 bits apart at qf_hb_off(f) = {0, 2, 8, 10}[f & 3] + 4 (f >> 2) and 16 above, so that one
// shift by 4 - {0, 2, 8, 10}[f & 3] serves a low pair (fields to bits 4, 20, above its nibbles)
// and a high pair (to bits 8, 24, above its 16-scaled nibbles).
__host__ __device__ __forceinline__ int qf_hb_off(int f) { return ((f & 1) << 1) + ((f & 2) << 2) + ((f >> 2) << 2); }
// The 5-bit types keep a record pair's fifth bits in one word: the even record's at the low bit
// of each Q6_K field position, the odd record's one above, so that shifting the word right by
// the record's parity turns it into a Q6_K word whose fields hold only their low bit.
// Bit position of the high 2 bits of record weight i.
__host__ __device__ __forceinline__ int qf_hb_pos(int i) {
    const int a = i & ~2, f = (a & 1) | (((a >> 2) & 1) << 1) | (((a >> 3) & 1) << 2);
    return qf_hb_off(f) + 16 * ((i >> 1) & 1);
}

// ------------------------------------------------------------------ weight arithmetic

// Scales of the f16 weight rules from the block fields (correctly rounded f16 products of exact
// operands): Q4_K (f16(d sc), f16(dmin m)), Q6_K f16(d sc).
__device__ __forceinline__ h16x2 q4k_scales(h16x2 d_dmin, h16x2 sc_m) { return d_dmin * sc_m; }
__device__ __forceinline__ h16 q6k_scale(h16 d, int sc) { return hmul(d, (h16)(float)sc); }
// Weight pairs from exact f16 pairs of quantized values: Q4_0 q - 8 (times d), Q4_K q (a q - b,
// one fused rounding), Q6_K q - 32 (times a).
__device__ __forceinline__ h16x2 q4_0_w2(h16x2 q8, h16x2 dd) { return q8 * dd; }
__device__ __forceinline__ h16x2 q4k_w2(h16x2 q, h16x2 aa, h16x2 nbb) { return __builtin_elementwise_fma(q, aa, nbb); }
__device__ __forceinline__ h16x2 q6k_w2(h16x2 q32, h16x2 aa) { return q32 * aa; }
// Q4_1 / Q5_1 weight pairs f16(f16(q d) + m): two roundings, the reference's f16 multiply then
// add (the library is built without multiply-add contraction).
__device__ __forceinline__ h16x2 q4_1_w2(h16x2 q, h16x2 dd, h16x2 mm) { return q * dd + mm; }

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
template <>
struct QRec<AESIR_GGML_Q4_1> {
    u32x2 nib;
    unsigned dm;  // f16 d | f16 m << 16
    unsigned hb;  // unused
};
template <>
struct QRec<AESIR_GGML_Q5_1> {
    u32x2 nib;
    unsigned dm;
    unsigned hb;  // the fifth bits, shifted to the even record's positions
};
template <>
struct QRec<AESIR_GGML_Q5_0> {
    u32x2 nib;
    h16 d;
    unsigned hb;
};
template <>
struct QRec<AESIR_GGML_Q5_K> {
    u32x2 nib;
    unsigned scm;
    unsigned dd;
    unsigned hb;
};
template <>
struct QRec<AESIR_GGML_Q2_K> {
    u32x2 nib;
    unsigned scm;  // GGML's byte: scale | min << 4
    unsigned dd;   // f16 d | f16 dmin << 16
};
template <>
struct QRec<AESIR_GGML_Q3_K> {
    u32x2 nib;
    int sc;
    h16 d;
};

// Record `rec` of plane row `prow`.
template <int T>
__device__ __forceinline__ QRec<T> qf_load(const QFMat &w, int64_t prow, int64_t rec, int64_t K) {
    QRec<T> q;
    if constexpr (qf_crumb<T>()) {
        const uint8_t *pr = (const uint8_t *)w.nib + qf_qlane_off(prow, rec, K, qf_lane_bytes(T));
        const unsigned c = *reinterpret_cast<const uint32_t *>(pr + 4 * (rec & 1));
        unsigned h = 0u;
        if constexpr (T == AESIR_GGML_Q3_K) h = *reinterpret_cast<const uint32_t *>(pr + 8) << (2 * (rec & 1));
        q.nib = crumb_nibbles(c, h);
    } else {
        q.nib = *reinterpret_cast<const u32x2 *>((const uint8_t *)w.nib + qf_nib_off(prow, rec, K));
    }
    const uint8_t *s0 = (const uint8_t *)w.s0 + qf_s0_off(prow, rec, K, qf_s0_bytes(T));
    if constexpr (qf_hb5<T>())
        q.hb = *reinterpret_cast<const uint32_t *>((const uint8_t *)w.hb + qf_hb_pair_off(prow, rec, K, 4)) >> (rec & 1);
    if constexpr (T == AESIR_GGML_Q4_0 || T == AESIR_GGML_Q5_0) {
        q.d = *reinterpret_cast<const h16 *>(s0);
    } else if constexpr (qf_dm<T>()) {
        q.dm = *reinterpret_cast<const uint32_t *>(s0);
    } else if constexpr (qf_kq<T>()) {
        q.scm = *reinterpret_cast<const uint16_t *>(s0);
        q.dd = *reinterpret_cast<const uint32_t *>((const uint8_t *)w.s1 + qf_s1_off(prow, rec, K, 4));
    } else if constexpr (T == AESIR_GGML_Q2_K) {
        q.scm = s0[rec & 1];
        q.dd = *reinterpret_cast<const uint32_t *>((const uint8_t *)w.s1 + qf_s1_off(prow, rec, K, 4));
    } else if constexpr (T == AESIR_GGML_Q3_K) {
        q.sc = *reinterpret_cast<const int8_t *>(s0 + (rec & 1));
        q.d = *reinterpret_cast<const h16 *>((const uint8_t *)w.s1 + qf_s1_off(prow, rec, K, 2));
    } else {
        q.hb = *reinterpret_cast<const uint32_t *>((const uint8_t *)w.hb + qf_hbw_off(prow, rec, K));
        q.sc = *reinterpret_cast<const int8_t *>(s0 + (rec & 1));
        q.d = *reinterpret_cast<const h16 *>((const uint8_t *)w.s1 + qf_s1_off(prow, rec, K, 2));
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
// The fifth bits of nibble pair f (value 16) from a 5-bit record's shifted word.
__device__ __forceinline__ unsigned qf_hb5_pair(unsigned hb, int f) {
    const int s = 4 - qf_hb_off(f);
    return (s >= 0 ? hb << s : hb >> -s) & 0x00100010u;
}

// Exact f16 pairs of the record's quantized values, pair order: Q4_0 q - 8, Q5_0 q - 16, Q4_1 /
// Q5_1 / Q4_K / Q5_K q, Q6_K q - 32.
template <int T>
__device__ __forceinline__ h16x2 qf_qpair(const QRec<T> &q, int f) {
    if constexpr (T == AESIR_GGML_Q4_0) {
        const h16x2 bias = {(h16)1032.0f, (h16)1032.0f};
        return as_h2(qf_pair(q.nib, f) | kMagic) - bias;
    } else if constexpr (qf_hb5<T>()) {
        const float b = T == AESIR_GGML_Q5_0 ? 1040.0f : 1024.0f;
        const h16x2 bias = {(h16)b, (h16)b};
        return as_h2(qf_pair(q.nib, f) | qf_hb5_pair(q.hb, f) | kMagic) - bias;
    } else if constexpr (T == AESIR_GGML_Q4_1 || T == AESIR_GGML_Q4_K || T == AESIR_GGML_Q2_K) {
        const h16x2 bias = {(h16)1024.0f, (h16)1024.0f};
        return as_h2(qf_pair(q.nib, f) | kMagic) - bias;
    } else if constexpr (T == AESIR_GGML_Q3_K) {
        const h16x2 bias = {(h16)1028.0f, (h16)1028.0f};
        return as_h2(qf_pair(q.nib, f) | kMagic) - bias;
    } else {
        const h16x2 bias = {(h16)1056.0f, (h16)1056.0f};
        return as_h2(qf_pair(q.nib, f) | qf_hb_pair(q.hb, f) | kMagic) - bias;
    }
}

// Natural-order weights from pair-order pairs: o[0] holds weights 0..7, o[1] 8..15.
__device__ __forceinline__ void qf_unpair(const unsigned (&wp)[8], u32x4 (&o)[2]) {
#pragma unroll
    for (int c = 0; c < 2; c++) {
        o[c].x = __builtin_amdgcn_perm(wp[4 * c + 1], wp[4 * c + 0], 0x05040100u);
        o[c].y = __builtin_amdgcn_perm(wp[4 * c + 1], wp[4 * c + 0], 0x07060302u);
        o[c].z = __builtin_amdgcn_perm(wp[4 * c + 3], wp[4 * c + 2], 0x05040100u);
        o[c].w = __builtin_amdgcn_perm(wp[4 * c + 3], wp[4 * c + 2], 0x07060302u);
    }
}

// The record's 16 f16 weights in natural order.
template <int T>
__device__ __forceinline__ void qf_deq16(const QRec<T> &q, u32x4 (&o)[2]) {
    unsigned wp[8];
    h16x2 aa, nbb;
    if constexpr (T == AESIR_GGML_Q4_0 || T == AESIR_GGML_Q5_0) {
        aa = h16x2{q.d, q.d};
    } else if constexpr (qf_dm<T>()) {
        const h16x2 dm = as_h2(q.dm);
        aa = h16x2{dm.x, dm.x};
        nbb = h16x2{dm.y, dm.y};  // the added min
    } else if constexpr (T == AESIR_GGML_Q2_K) {
        const h16x2 ab = q4k_scales(as_h2(q.dd), h16x2{(h16)(float)(q.scm & 15u), (h16)(float)(q.scm >> 4)});
        aa = h16x2{ab.x, ab.x};
        nbb = h16x2{-ab.y, -ab.y};
    } else if constexpr (T == AESIR_GGML_Q3_K) {
        const h16 a = q6k_scale(q.d, q.sc);
        aa = h16x2{a, a};
    } else if constexpr (qf_kq<T>()) {
        const h16x2 sm = {(h16)(float)(q.scm & 0xffu), (h16)(float)(q.scm >> 8)};
        const h16x2 ab = q4k_scales(as_h2(q.dd), sm);
        aa = h16x2{ab.x, ab.x};
        nbb = h16x2{-ab.y, -ab.y};
    } else {
        const h16 a = q6k_scale(q.d, q.sc);
        aa = h16x2{a, a};
    }
#pragma unroll
    for (int f = 0; f < 8; f++) {
        const h16x2 v = qf_qpair(q, f);
        if constexpr (T == AESIR_GGML_Q4_0 || T == AESIR_GGML_Q5_0) wp[f] = h2_bits(q4_0_w2(v, aa));
        else if constexpr (qf_dm<T>()) wp[f] = h2_bits(q4_1_w2(v, aa, nbb));
        else if constexpr (qf_kq<T>() || T == AESIR_GGML_Q2_K) wp[f] = h2_bits(q4k_w2(v, aa, nbb));
        else wp[f] = h2_bits(q6k_w2(v, aa));
    }
    qf_unpair(wp, o);
}

// ------------------------------------------------------------------ repacking

// GGUF source of weight e of a row: its 4- or 6-bit value.
template <int T>
__device__ __forceinline__ int gguf_q(const uint8_t *row, int64_t e) {
    if constexpr (T == AESIR_GGML_Q4_0) {
        const uint8_t *blk = row + (e / 32) * 18;
        const int i = (int)(e % 32);
        return i < 16 ? (blk[2 + i] & 15) : (blk[2 + i - 16] >> 4);
    } else if constexpr (T == AESIR_GGML_Q8_0) {
        return (int)(int8_t)row[(e / 32) * 34 + 2 + e % 32];
    } else if constexpr (T == AESIR_GGML_Q4_1 || T == AESIR_GGML_Q5_0 || T == AESIR_GGML_Q5_1) {
        // {d, (m), (qh[4]), qs[16]}: nibbles as Q4_0, bit i of the qh word the fifth bit
        constexpr int bb = T == AESIR_GGML_Q4_1 ? 20 : T == AESIR_GGML_Q5_0 ? 22 : 24;
        constexpr int qs = T == AESIR_GGML_Q5_0 ? 6 : T == AESIR_GGML_Q4_1 ? 4 : 8;
        const uint8_t *blk = row + (e / 32) * bb;
        const int i = (int)(e % 32);
        const int q = i < 16 ? (blk[qs + i] & 15) : (blk[qs + i - 16] >> 4);
        if constexpr (T == AESIR_GGML_Q4_1) return q;
        else return q | (((blk[qs - 4 + i / 8] >> (i % 8)) & 1) << 4);
    } else if constexpr (T == AESIR_GGML_Q5_K) {
        const uint8_t *blk = row + (e / 256) * 176, *qh = blk + 16, *qs = blk + 48;
        const int i = (int)(e % 256), g = i / 64, hi = (i / 32) & 1, l = i % 32;
        const int q = hi ? (qs[32 * g + l] >> 4) : (qs[32 * g + l] & 15);
        return q | (((qh[l] >> (2 * g + hi)) & 1) << 4);
    } else if constexpr (T == AESIR_GGML_Q2_K || T == AESIR_GGML_Q3_K) {
        // 2-bit values of half h, shift j, position l; Q3_K less 4 unless its hmask bit is set
        const int i = (int)(e % 256), h = i / 128, j = (i / 32) & 3, l = i % 32;
        if constexpr (T == AESIR_GGML_Q2_K) {
            return (row[(e / 256) * 84 + 16 + 32 * h + l] >> (2 * j)) & 3;
        } else {
            const uint8_t *blk = row + (e / 256) * 110;
            return ((blk[32 + 32 * h + l] >> (2 * j)) & 3) - ((blk[l] >> (4 * h + j)) & 1 ? 0 : 4);
        }
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

__device__ __forceinline__ int64_t gguf_row_bytes(int T, int64_t K) {
    switch (T) {
        case AESIR_GGML_Q4_0: return K / 32 * 18;
        case AESIR_GGML_Q4_1: return K / 32 * 20;
        case AESIR_GGML_Q5_0: return K / 32 * 22;
        case AESIR_GGML_Q5_1: return K / 32 * 24;
        case AESIR_GGML_Q8_0: return K / 32 * 34;
        case AESIR_GGML_Q2_K: return K / 256 * 84;
        case AESIR_GGML_Q3_K: return K / 256 * 110;
        case AESIR_GGML_Q4_K: return K / 256 * 144;
        case AESIR_GGML_Q5_K: return K / 256 * 176;
        default: return K / 256 * 210;
    }
}

// 16-weight sub-block `is` (0..15) scale of a Q3_K super-block: GGML's packing of 16 6-bit values
// in 12 bytes (low 4 bits in bytes 0-7, low then high nibble; high 2 bits in bytes 8-11), less 32.
__device__ __forceinline__ int q3k_scale(const uint8_t *sc, int is) {
    const int lo = is < 8 ? (sc[is] & 15) : (sc[is - 8] >> 4);
    return (lo | (((sc[8 + (is & 3)] >> (2 * (is >> 2))) & 3) << 4)) - 32;
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
    const uint8_t *src = blocks + r * gguf_row_bytes(T, K);
    const int64_t prow = dst.row0 + r * step;
    int q[kRec];
#pragma unroll
    for (int i = 0; i < kRec; i++) q[i] = gguf_q<T>(src, k + i) + (T == AESIR_GGML_Q3_K ? 4 : 0);  // Q3_K: 0..7
    unsigned nib[2] = {0u, 0u}, hb = 0u;
#pragma unroll
    for (int j = 0; j < 8; j++) nib[j >> 2] |= (unsigned)((q[j] & 15) | ((q[8 + j] & 15) << 4)) << (8 * (j & 3));
    if constexpr (T == AESIR_GGML_Q6_K) {
#pragma unroll
        for (int i = 0; i < kRec; i++) hb |= (unsigned)(q[i] >> 4) << qf_hb_pos(i);
        *reinterpret_cast<uint32_t *>((uint8_t *)dst.hb + qf_hbw_off(prow, rec, K)) = hb;
    }
    if constexpr (qf_hb5<T>()) {  // the even record writes the pair's word (its bits and the odd record's)
        if (rec % 2 == 0) {
#pragma unroll
            for (int i = 0; i < kRec; i++) {
                hb |= (unsigned)((q[i] >> 4) & 1) << qf_hb_pos(i);
                hb |= (unsigned)((gguf_q<T>(src, k + kRec + i) >> 4) & 1) << (qf_hb_pos(i) + 1);
            }
            *reinterpret_cast<uint32_t *>((uint8_t *)dst.hb + qf_hb_pair_off(prow, rec, K, 4)) = hb;
        }
    }
    if constexpr (qf_crumb<T>()) {
        uint8_t *pr = (uint8_t *)dst.nib + qf_qlane_off(prow, rec, K, qf_lane_bytes(T));
        *reinterpret_cast<uint32_t *>(pr + 4 * (rec & 1)) = crumb_word(nib[0], nib[1]);
        if constexpr (T == AESIR_GGML_Q3_K) {
            if (rec % 2 == 0) {  // the even record writes the pair's third bits (its own and the odd record's)
                unsigned nib1[2] = {0u, 0u};
#pragma unroll
                for (int j = 0; j < 8; j++)
                    nib1[j >> 2] |= (unsigned)((gguf_q<T>(src, k + kRec + j) + 4) | ((gguf_q<T>(src, k + kRec + 8 + j) + 4) << 4))
                                    << (8 * (j & 3));
                *reinterpret_cast<uint32_t *>(pr + 8) = third_bits(nib[0], nib[1], 0) | third_bits(nib1[0], nib1[1], 1);
            }
        }
    } else {
        *reinterpret_cast<u32x2 *>((uint8_t *)dst.nib + qf_nib_off(prow, rec, K)) = u32x2{nib[0], nib[1]};
    }
    uint8_t *s0 = (uint8_t *)dst.s0 + qf_s0_off(prow, rec, K, qf_s0_bytes(T));
    if constexpr (T == AESIR_GGML_Q4_0 || T == AESIR_GGML_Q5_0 || qf_dm<T>()) {
        if (rec % 2 == 0) {  // the block's f16 d (and m), the first 2 (4) bytes of every legacy block
            const uint8_t *blk = src + (k / 32) * (gguf_row_bytes(T, 32));
            if constexpr (qf_dm<T>())
                *reinterpret_cast<uint32_t *>(s0) = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8) | ((uint32_t)blk[2] << 16) |
                                                    ((uint32_t)blk[3] << 24);
            else
                *reinterpret_cast<uint16_t *>(s0) = (uint16_t)(blk[0] | (blk[1] << 8));
        }
    } else if constexpr (T == AESIR_GGML_Q2_K || T == AESIR_GGML_Q3_K) {
        // the record's 16-weight sub-block: its scale byte (Q2_K: scale | min << 4 as GGML packs
        // it; Q3_K: the unpacked signed scale), and the super-block's d (and dmin)
        const int i = (int)(k % 256), is = 8 * (i / 128) + 2 * ((i / 32) & 3) + ((i / 16) & 1);
        if constexpr (T == AESIR_GGML_Q2_K) {
            const uint8_t *blk = src + (k / 256) * 84;
            s0[rec & 1] = blk[is];
            if (rec % 16 == 0)
                *reinterpret_cast<uint32_t *>((uint8_t *)dst.s1 + qf_s1_off(prow, rec, K, 4)) =
                    (uint32_t)blk[80] | ((uint32_t)blk[81] << 8) | ((uint32_t)blk[82] << 16) | ((uint32_t)blk[83] << 24);
        } else {
            const uint8_t *blk = src + (k / 256) * 110;
            s0[rec & 1] = (uint8_t)(int8_t)q3k_scale(blk + 96, is);
            if (rec % 16 == 0)
                *reinterpret_cast<uint16_t *>((uint8_t *)dst.s1 + qf_s1_off(prow, rec, K, 2)) =
                    (uint16_t)(blk[108] | (blk[109] << 8));
        }
    } else if constexpr (qf_kq<T>()) {
        const uint8_t *blk = src + (k / 256) * (T == AESIR_GGML_Q4_K ? 144 : 176);
        if (rec % 2 == 0) {
            int s, m;
            q4k_scale_min(blk + 4, (int)((k % 256) / 32), s, m);
            *reinterpret_cast<uint16_t *>(s0) = (uint16_t)(s | (m << 8));
        }
        if (rec % 16 == 0)
            *reinterpret_cast<uint32_t *>((uint8_t *)dst.s1 + qf_s1_off(prow, rec, K, 4)) =
                (uint32_t)blk[0] | ((uint32_t)blk[1] << 8) | ((uint32_t)blk[2] << 16) | ((uint32_t)blk[3] << 24);
    } else {
        const uint8_t *blk = src + (k / 256) * 210;
        s0[rec & 1] = blk[192 + (k % 256) / 16];
        if (rec % 16 == 0)
            *reinterpret_cast<uint16_t *>((uint8_t *)dst.s1 + qf_s1_off(prow, rec, K, 2)) =
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
    qf_deq16<T>(qf_load<T>(w, w.row0 + src_row * step, rec, K), o);
    h16 *dst = out + r * out_stride + rec * kRec;
    st16(dst, o[0]);
    st16(dst + 8, o[1]);
}

// One thread per record: GGUF blocks -> f16 weights straight from the blocks, with the same
// weight rules (and instructions) as qf_deq16 (the f16 route of aesir_gemm_quant, and the parts of
// a fused model matrix stored in f16).
template <int T>
__global__ __launch_bounds__(256) void gguf_dequant_kernel(const uint8_t *__restrict__ blocks, int64_t rows, int64_t K,
                                                           h16 *__restrict__ out, int64_t out_stride) {
    const int64_t recs = K / kRec;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= rows * recs) return;
    const int64_t r = gid / recs, rec = gid % recs, k = rec * kRec;
    const uint8_t *src = blocks + r * gguf_row_bytes(T, K);
    auto f16_at = [](const uint8_t *p) { return bits_to_h((uint16_t)(p[0] | (p[1] << 8))); };
    h16x2 aa, nbb;  // the record's scale pair and negated offset (or added min) pair
    if constexpr (T == AESIR_GGML_Q4_0 || T == AESIR_GGML_Q8_0 || T == AESIR_GGML_Q5_0) {
        const h16 d = f16_at(src + (k / 32) * (T == AESIR_GGML_Q4_0 ? 18 : T == AESIR_GGML_Q8_0 ? 34 : 22));
        aa = h16x2{d, d};
    } else if constexpr (T == AESIR_GGML_Q4_1 || T == AESIR_GGML_Q5_1) {
        const uint8_t *blk = src + (k / 32) * (T == AESIR_GGML_Q4_1 ? 20 : 24);
        aa = h16x2{f16_at(blk), f16_at(blk)};
        nbb = h16x2{f16_at(blk + 2), f16_at(blk + 2)};
    } else if constexpr (T == AESIR_GGML_Q4_K || T == AESIR_GGML_Q5_K || T == AESIR_GGML_Q2_K) {
        int s, m;
        const uint8_t *dm;
        if constexpr (T == AESIR_GGML_Q2_K) {
            const uint8_t *blk = src + (k / 256) * 84;
            const int i = (int)(k % 256), is = 8 * (i / 128) + 2 * ((i / 32) & 3) + (i / 16 & 1);
            s = blk[is] & 15;
            m = blk[is] >> 4;
            dm = blk + 80;
        } else {
            const uint8_t *blk = src + (k / 256) * (T == AESIR_GGML_Q4_K ? 144 : 176);
            q4k_scale_min(blk + 4, (int)((k % 256) / 32), s, m);
            dm = blk;
        }
        const h16x2 ab = q4k_scales(h16x2{f16_at(dm), f16_at(dm + 2)}, h16x2{(h16)(float)s, (h16)(float)m});
        aa = h16x2{ab.x, ab.x};
        nbb = h16x2{-ab.y, -ab.y};
    } else if constexpr (T == AESIR_GGML_Q3_K) {
        const uint8_t *blk = src + (k / 256) * 110;
        const int i = (int)(k % 256), is = 8 * (i / 128) + 2 * ((i / 32) & 3) + (i / 16 & 1);
        const h16 a = q6k_scale(f16_at(blk + 108), q3k_scale(blk + 96, is));
        aa = h16x2{a, a};
    } else {
        const uint8_t *blk = src + (k / 256) * 210;
        const h16 a = q6k_scale(f16_at(blk + 208), (int8_t)blk[192 + (k % 256) / 16]);
        aa = h16x2{a, a};
    }
    unsigned wp[8];  // natural pairs (2 i, 2 i + 1)
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int q0 = gguf_q<T>(src, k + 2 * i), q1 = gguf_q<T>(src, k + 2 * i + 1);
        auto pair = [](int a, int b) { return h16x2{(h16)(float)a, (h16)(float)b}; };
        if constexpr (T == AESIR_GGML_Q4_0)
            wp[i] = h2_bits(q4_0_w2(pair(q0 - 8, q1 - 8), aa));
        else if constexpr (T == AESIR_GGML_Q5_0)
            wp[i] = h2_bits(q4_0_w2(pair(q0 - 16, q1 - 16), aa));
        else if constexpr (T == AESIR_GGML_Q8_0)  // f16(f16(q) * d), as the Q8_0 GEMV
            wp[i] = h2_bits(h16x2{(h16)((float)q0 * (float)aa.x), (h16)((float)q1 * (float)aa.x)});
        else if constexpr (T == AESIR_GGML_Q4_1 || T == AESIR_GGML_Q5_1)
            wp[i] = h2_bits(q4_1_w2(pair(q0, q1), aa, nbb));
        else if constexpr (T == AESIR_GGML_Q4_K || T == AESIR_GGML_Q5_K || T == AESIR_GGML_Q2_K)
            wp[i] = h2_bits(q4k_w2(pair(q0, q1), aa, nbb));
        else if constexpr (T == AESIR_GGML_Q3_K)
            wp[i] = h2_bits(q6k_w2(pair(q0, q1), aa));
        else
            wp[i] = h2_bits(q6k_w2(pair(q0 - 32, q1 - 32), aa));
    }
    h16 *dst = out + r * out_stride + k;
    st16(dst, u32x4{wp[0], wp[1], wp[2], wp[3]});
    st16(dst + 8, u32x4{wp[4], wp[5], wp[6], wp[7]});
}

// One thread per record: uniform random values; scales chosen so that the weights have a
// standard deviation near `std` and a mean near 0. The values depend on (row, record) only, not
// on where the planes put them.
template <int T>
__global__ __launch_bounds__(256) void qf_fill_kernel(QFMat w, int64_t rows, int64_t K, int64_t step, uint64_t base,
                                                      float std) {
    const int64_t recs = K / kRec;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= rows * recs) return;
    const int64_t r = gid / recs, rec = gid % recs, prow = w.row0 + r * step;
    const uint64_t a = mix64(base + (uint64_t)(2 * gid + 1) * kGolden);
    const uint64_t b = mix64(base + (uint64_t)(2 * gid + 2) * kGolden);
    if constexpr (qf_crumb<T>()) {
        // Q2_K / Q3_K: 16 uniform crumbs; Q3_K's pair word of uniform third bits (even record)
        uint8_t *pr = (uint8_t *)w.nib + qf_qlane_off(prow, rec, K, qf_lane_bytes(T));
        *reinterpret_cast<uint32_t *>(pr + 4 * (rec & 1)) = (unsigned)a;
        if constexpr (T == AESIR_GGML_Q3_K)
            if (rec % 2 == 0) *reinterpret_cast<uint32_t *>(pr + 8) = (unsigned)(a >> 32);
    } else {
        *reinterpret_cast<u32x2 *>((uint8_t *)w.nib + qf_nib_off(prow, rec, K)) = u32x2{(unsigned)a, (unsigned)(a >> 32)};
    }
    uint8_t *s0 = (uint8_t *)w.s0 + qf_s0_off(prow, rec, K, qf_s0_bytes(T));
    const float u = (float)(b >> 40) * (1.0f / 16777216.0f);  // [0, 1)
    // 5-bit types: uniform fifth bits, one word per record pair (written by the even record)
    if constexpr (qf_hb5<T>())
        if (rec % 2 == 0) *reinterpret_cast<uint32_t *>((uint8_t *)w.hb + qf_hb_pair_off(prow, rec, K, 4)) = (uint32_t)(b >> 8);
    constexpr float qsd = qf_hb5<T>() ? 9.23f : 4.61f;  // standard deviation of q uniform on [0, 31] / [0, 15]
    constexpr float qmid = qf_hb5<T>() ? 15.5f : 7.5f;
    if constexpr (T == AESIR_GGML_Q4_0 || T == AESIR_GGML_Q5_0) {
        // q - 8 (q - 16) uniform on [-8, 7] ([-16, 15])
        if (rec % 2 == 0) *reinterpret_cast<h16 *>(s0) = (h16)((0.5f + u) * std / qsd);
    } else if constexpr (qf_dm<T>()) {
        // m = -f16(qmid d): w = q d + m centred near 0
        if (rec % 2 == 0) {
            const h16 d = (h16)((0.5f + u) * std / qsd), m = (h16)(-qmid * (float)d);
            *reinterpret_cast<uint32_t *>(s0) = (uint32_t)h_to_bits(d) | ((uint32_t)h_to_bits(m) << 16);
        }
    } else if constexpr (T == AESIR_GGML_Q2_K) {
        // q uniform on [0, 3] (standard deviation 1.118); sc in [4, 8], m = round(1.5 sc), dmin = d
        const int sc = 4 + (int)((b >> 8) % 5), m = (int)(1.5f * (float)sc + 0.5f);
        s0[rec & 1] = (uint8_t)(sc | (m << 4));
        if (rec % 16 == 0) {
            const uint32_t dv = h_to_bits((h16)((0.5f + u) * std / (6.0f * 1.118f)));
            *reinterpret_cast<uint32_t *>((uint8_t *)w.s1 + qf_s1_off(prow, rec, K, 4)) = dv | (dv << 16);
        }
    } else if constexpr (T == AESIR_GGML_Q3_K) {
        // q - 4 uniform on [-4, 3] (standard deviation 2.29); sc in [16, 31]
        s0[rec & 1] = (uint8_t)(16 + (int)((b >> 4) % 16));
        if (rec % 16 == 0)
            *reinterpret_cast<h16 *>((uint8_t *)w.s1 + qf_s1_off(prow, rec, K, 2)) = (h16)((0.5f + u) * std / (24.0f * 2.29f));
    } else if constexpr (qf_kq<T>()) {
        // sc in [4, 8], m = round(qmid sc / mk), dmin = mk d: w = d sc (q - qmid) nearly, m within
        // the 6 bits GGML's packing holds
        constexpr float mk = T == AESIR_GGML_Q5_K ? 2.0f : 1.0f;
        if (rec % 2 == 0) {
            const int s = 4 + (int)((b >> 8) % 5), m = (int)(qmid * (float)s / mk + 0.5f);
            *reinterpret_cast<uint16_t *>(s0) = (uint16_t)(s | (m << 8));
        }
        if (rec % 16 == 0) {
            const h16 d = (h16)((0.5f + u) * std / (6.0f * qsd));
            const uint32_t dv = h_to_bits(d), mv = h_to_bits((h16)(mk * (float)d));
            *reinterpret_cast<uint32_t *>((uint8_t *)w.s1 + qf_s1_off(prow, rec, K, 4)) = dv | (mv << 16);
        }
    } else {
        // q - 32 uniform on [-32, 31]: standard deviation 18.5; sc in [16, 47]
        *reinterpret_cast<uint32_t *>((uint8_t *)w.hb + qf_hbw_off(prow, rec, K)) = (uint32_t)(b >> 8);
        s0[rec & 1] = (uint8_t)(16 + (int)((b >> 4) % 32));
        if (rec % 16 == 0)
            *reinterpret_cast<h16 *>((uint8_t *)w.s1 + qf_s1_off(prow, rec, K, 2)) =
                (h16)((0.5f + u) * std / (32.0f * 18.5f));
    }
}

static unsigned rec_grid(int64_t rows, int64_t K) { return (unsigned)((rows * (K / kRec) + 255) / 256); }

static int32_t qf_check(int32_t type, int64_t K, const char *name) {
    if (!qf_type(type))
        return fail(AESIR_ERR_UNSUPPORTED,
                    "%s: weight type %d is not Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q4_K, Q5_K or Q6_K", name, (int)type);
    const int64_t blk = gguf_block_elems(type);
    if (K <= 0 || K % blk != 0)
        return fail(AESIR_ERR_SHAPE, "%s: row length %lld is not a multiple of the %lld-weight block", name, (long long)K,
                    (long long)blk);
    return AESIR_OK;
}

// Runs F<T>() for the repacked type `type` (one of qf_type's).
template <class F>
static void qf_switch(int32_t type, F &&f) {
    switch (type) {
        case AESIR_GGML_Q4_0: f(std::integral_constant<int, AESIR_GGML_Q4_0>{}); break;
        case AESIR_GGML_Q4_1: f(std::integral_constant<int, AESIR_GGML_Q4_1>{}); break;
        case AESIR_GGML_Q5_0: f(std::integral_constant<int, AESIR_GGML_Q5_0>{}); break;
        case AESIR_GGML_Q5_1: f(std::integral_constant<int, AESIR_GGML_Q5_1>{}); break;
        case AESIR_GGML_Q2_K: f(std::integral_constant<int, AESIR_GGML_Q2_K>{}); break;
        case AESIR_GGML_Q3_K: f(std::integral_constant<int, AESIR_GGML_Q3_K>{}); break;
        case AESIR_GGML_Q4_K: f(std::integral_constant<int, AESIR_GGML_Q4_K>{}); break;
        case AESIR_GGML_Q5_K: f(std::integral_constant<int, AESIR_GGML_Q5_K>{}); break;
        default: f(std::integral_constant<int, AESIR_GGML_Q6_K>{}); break;
    }
}

// The tiled planes need whole 128-weight segments.
static int32_t qf_check_planes(int32_t type, int64_t K, const char *name) {
    AESIR_TRY(qf_check(type, K, name));
    if (K % kSeg != 0)
        return fail(AESIR_ERR_UNSUPPORTED, "%s: repacked planes need a row length that is a multiple of 128 (got %lld)",
                    name, (long long)K);
    return AESIR_OK;
}

int32_t launch_qf_repack(hipStream_t s, int32_t type, const void *blocks, int64_t rows, int64_t K, const QFMat &dst,
                         int64_t step) {
    AESIR_TRY(qf_check_planes(type, K, "repack"));
    if (rows <= 0) return AESIR_OK;
    const unsigned g = rec_grid(rows, K);
    qf_switch(type, [&](auto t) {
        hipLaunchKernelGGL(qf_repack_kernel<decltype(t)::value>, dim3(g), dim3(256), 0, s, (const uint8_t *)blocks, rows,
                           K, dst, step);
    });
    AESIR_LAUNCH_CHECK("qf_repack_kernel");
    return AESIR_OK;
}

int32_t launch_qf_dequant(hipStream_t s, const QFMat &w, int64_t rows, int64_t K, int64_t step,
                          const int64_t *row_ids, void *out, int64_t out_stride) {
    AESIR_TRY(qf_check_planes(w.type, K, "dequant"));
    if (rows <= 0) return AESIR_OK;
    const unsigned g = rec_grid(rows, K);
    qf_switch(w.type, [&](auto t) {
        hipLaunchKernelGGL(qf_dequant_kernel<decltype(t)::value>, dim3(g), dim3(256), 0, s, w, rows, K, step, row_ids,
                           (h16 *)out, out_stride);
    });
    AESIR_LAUNCH_CHECK("qf_dequant_kernel");
    return AESIR_OK;
}

int64_t gguf_block_elems(int32_t type) {
    switch (type) {
        case AESIR_GGML_Q4_0:
        case AESIR_GGML_Q4_1:
        case AESIR_GGML_Q5_0:
        case AESIR_GGML_Q5_1:
        case AESIR_GGML_Q8_0: return 32;
        case AESIR_GGML_Q2_K:
        case AESIR_GGML_Q3_K:
        case AESIR_GGML_Q4_K:
        case AESIR_GGML_Q5_K:
        case AESIR_GGML_Q6_K: return 256;
        default: return 0;
    }
}

int32_t launch_gguf_dequant(hipStream_t s, int32_t type, const void *blocks, int64_t rows, int64_t K, void *out,
                            int64_t out_stride) {
    const int64_t blk = gguf_block_elems(type);
    if (blk == 0) return fail(AESIR_ERR_UNSUPPORTED, "gguf_dequant: GGML type %d is not a block type of this library", (int)type);
    if (K <= 0 || K % blk != 0)
        return fail(AESIR_ERR_SHAPE, "gguf_dequant: row length %lld is not a multiple of the %lld-weight block",
                    (long long)K, (long long)blk);
    if (out_stride < K || out_stride % 8 != 0 || ((uintptr_t)out & 15) != 0)
        return fail(AESIR_ERR_SHAPE, "gguf_dequant: output rows must be 16-byte aligned and hold K weights");
    if (rows <= 0) return AESIR_OK;
    const unsigned g = rec_grid(rows, K);
    const uint8_t *b = (const uint8_t *)blocks;
    h16 *o = (h16 *)out;
#define AESIR_GD(TY)                                                                                               \
    case TY: hipLaunchKernelGGL(gguf_dequant_kernel<TY>, dim3(g), dim3(256), 0, s, b, rows, K, o, out_stride); break
    switch (type) {
        AESIR_GD(AESIR_GGML_Q4_0);
        AESIR_GD(AESIR_GGML_Q4_1);
        AESIR_GD(AESIR_GGML_Q5_0);
        AESIR_GD(AESIR_GGML_Q5_1);
        AESIR_GD(AESIR_GGML_Q8_0);
        AESIR_GD(AESIR_GGML_Q2_K);
        AESIR_GD(AESIR_GGML_Q3_K);
        AESIR_GD(AESIR_GGML_Q4_K);
        AESIR_GD(AESIR_GGML_Q5_K);
        AESIR_GD(AESIR_GGML_Q6_K);
        default: break;
    }
#undef AESIR_GD
    AESIR_LAUNCH_CHECK("gguf_dequant_kernel");
    return AESIR_OK;
}

int32_t launch_qf_fill_random(hipStream_t s, const QFMat &w, int64_t rows, int64_t K, int64_t step, uint64_t seed,
                              uint64_t stream, float std) {
    AESIR_TRY(qf_check_planes(w.type, K, "fill"));
    if (rows <= 0) return AESIR_OK;
    const uint64_t base = mix64(seed ^ mix64(stream + kGolden));
    const unsigned g = rec_grid(rows, K);
    qf_switch(w.type, [&](auto t) {
        hipLaunchKernelGGL(qf_fill_kernel<decltype(t)::value>, dim3(g), dim3(256), 0, s, w, rows, K, step, base, std);
    });
    AESIR_LAUNCH_CHECK("qf_fill_kernel");
    return AESIR_OK;
}

// ------------------------------------------------------------------ decode GEMV (matrix cores)

// Work of a workgroup: 16-row blocks blockIdx.x, + gridDim.x, ... (one block per workgroup when
// the blocks are few, 256 persistent workgroups looping over them when there are many); wave w
// multiplies a block's tiles of segments w, w + NW, ..., in rounds of qf_round() tiles whose loads
// are issued together, the next round's (of this block or the next) while the current one
// computes. Each lane dequantizes its 32 weights of a tile (two records of row lane % 16) into
// four A operands, and x, staged once per workgroup in LDS in the matching pair order, is the B
// operand, the same in all 16 columns, so every column of the 16 x 16 accumulator holds the row
// sums. Per tile and lane: one 16-byte nibble load, 4 matrix-core steps, and the dequantization
// (Q4_0 / Q4_K 52, Q6_K 76 VALU instructions). Q6_K tiles hold twice the registers (high-bit
// words, wider dequantization), so their rounds are half as long.
template <int T>
constexpr int qf_round() {
    return T == AESIR_GGML_Q6_K ? 2 : 4;
}

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
    unsigned flo, fhi;       // fifth-bit masks 0x00100010 / 0x01000100
    __device__ __forceinline__ static QfRegs make() {
        return QfRegs{sreg(0x000F000Fu), sreg(0x00F000F0u), vreg(kMagic), sreg(0x00300030u),
                      sreg(0x03000300u), sreg(0x00100010u), sreg(0x01000100u)};
    }
};

// One lane's share of a tile as loaded.
template <int T>
struct QTile;
template <>
struct QTile<AESIR_GGML_Q4_0> {
    u32x4 nib;
    unsigned s0;  // f16 d in the low half
};
template <>
struct QTile<AESIR_GGML_Q4_K> {
    u32x4 nib;
    unsigned s0;  // scale | min << 8
    unsigned s1;  // f16 d | f16 dmin << 16
};
template <>
struct QTile<AESIR_GGML_Q6_K> {
    u32x4 nib;
    u32x2 hb;     // high-bit words of the two records
    unsigned s0;  // int8 scales of the two records
    unsigned s1;  // f16 super-block d in the low half
};
template <>
struct QTile<AESIR_GGML_Q5_0> {
    u32x4 nib;
    unsigned s0;  // f16 d in the low half
    unsigned hb;  // fifth bits of the two records
};
template <>
struct QTile<AESIR_GGML_Q4_1> {
    u32x4 nib;
    unsigned s0;  // f16 d | f16 m << 16
};
template <>
struct QTile<AESIR_GGML_Q5_1> {
    u32x4 nib;
    unsigned s0;  // f16 d | f16 m << 16
    unsigned hb;
};
template <>
struct QTile<AESIR_GGML_Q5_K> {
    u32x4 nib;
    unsigned s0;  // scale | min << 8
    unsigned s1;  // f16 d | f16 dmin << 16
    unsigned hb;
};
template <>
struct QTile<AESIR_GGML_Q2_K> {
    u32x2 cr;     // crumb words of the two records
    unsigned s0;  // the two records' scale | min << 4 bytes
    unsigned s1;  // f16 d | f16 dmin << 16
};
template <>
struct QTile<AESIR_GGML_Q3_K> {
    u32x2 cr;     // crumb words of the two records
    unsigned hb;  // third bits of the record pair
    unsigned s0;  // int8 scales of the two records
    unsigned s1;  // f16 super-block d in the low half
};

// Buffer resources of a matrix's planes (range-checked loads, tile offsets in SGPRs).
struct QfRsrc {
    __amdgpu_buffer_rsrc_t nib, hb, s0, s1;
};

__device__ __forceinline__ QfRsrc qf_rsrc(const QFMat &w, int32_t type, int64_t prows, int64_t K) {
    QfRsrc r;
    r.nib = __builtin_amdgcn_make_buffer_rsrc((void *)w.nib, 0, (int)(prows * qf_plane_row_bytes(type, 0, K)), 0x00020000);
    r.hb = __builtin_amdgcn_make_buffer_rsrc((void *)w.hb, 0, (int)(prows * qf_plane_row_bytes(type, 1, K)), 0x00020000);
    r.s0 = __builtin_amdgcn_make_buffer_rsrc((void *)w.s0, 0, (int)(prows * qf_plane_row_bytes(type, 2, K)), 0x00020000);
    r.s1 = __builtin_amdgcn_make_buffer_rsrc((void *)w.s1, 0, (int)(prows * qf_plane_row_bytes(type, 3, K)), 0x00020000);
    return r;
}

// Tile `tile` (wave-uniform); s1v / s1s: the lane's and the tile's byte offsets in the s1 plane.
template <int T>
__device__ __forceinline__ QTile<T> qf_tile_load(const QfRsrc &r, int tile, int lane, int s1v, int s1s) {
    QTile<T> q;
    if constexpr (T == AESIR_GGML_Q2_K) {
        q.cr = __builtin_amdgcn_raw_buffer_load_b64(r.nib, lane * 8, tile * 512, 2);
    } else if constexpr (T == AESIR_GGML_Q3_K) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b96(r.nib, lane * 12, tile * 768, 2);
        q.cr = u32x2{(unsigned)v[0], (unsigned)v[1]};
        q.hb = (unsigned)v[2];
    } else {
        q.nib = __builtin_amdgcn_raw_buffer_load_b128(r.nib, lane * 16, tile * 1024, 2);
    }
    if constexpr (qf_dm<T>())
        q.s0 = __builtin_amdgcn_raw_buffer_load_b32(r.s0, lane * 4, tile * 256, 0);
    else
        q.s0 = __builtin_amdgcn_raw_buffer_load_b16(r.s0, lane * 2, tile * 128, 0);
    if constexpr (qf_hb5<T>()) q.hb = __builtin_amdgcn_raw_buffer_load_b32(r.hb, lane * 4, tile * 256, 0);
    if constexpr (qf_kq<T>() || T == AESIR_GGML_Q2_K) q.s1 = __builtin_amdgcn_raw_buffer_load_b32(r.s1, s1v, s1s, 0);
    if constexpr (T == AESIR_GGML_Q3_K) q.s1 = __builtin_amdgcn_raw_buffer_load_b16(r.s1, s1v, s1s, 0);
    if constexpr (T == AESIR_GGML_Q6_K) {
        q.hb = __builtin_amdgcn_raw_buffer_load_b64(r.hb, lane * 8, tile * 512, 2);
        q.s1 = __builtin_amdgcn_raw_buffer_load_b16(r.s1, s1v, s1s, 0);
    }
    return q;
}

// The four A operands of a lane's tile share: operand j from nibble word j (record j / 2, bytes
// 4 (j % 2) .. + 3), as the pairs (v & lo), (v >> 8 & lo), (v & hi), (v >> 8 & hi), i.e. the
// weights {0, 2, 1, 3, 8, 10, 9, 11} + 4 (j % 2) of the record. Values exact in f16 until the
// weight rule's single rounding: Q4_0 turns 1024 + q into q - 8 by adding -1032 and 1024 + 16 q
// by (.) / 16 - 72; Q4_K into q by -1024 and (.) / 16 - 64; Q6_K into q - 32 by -1056 and
// (.) / 16 - 96, its high bits OR-ed in from the record's hb word (shifted by 4, 2, -4, -6 for
// the four pair positions of the record).
template <int T>
__device__ __forceinline__ void qf_tile_a(const QTile<T> &q, const QfRegs &k, u32x4 (&a)[4]) {
    unsigned nw[4];
    if constexpr (qf_crumb<T>()) {  // spread the crumbs (and Q3_K's third bits) into nibble words
        unsigned h = 0u;
        if constexpr (T == AESIR_GGML_Q3_K) h = q.hb;
        const u32x2 e = crumb_nibbles(q.cr.x, h), o = crumb_nibbles(q.cr.y, h << 2);
        nw[0] = e.x;
        nw[1] = e.y;
        nw[2] = o.x;
        nw[3] = o.y;
    } else {
        nw[0] = q.nib.x;
        nw[1] = q.nib.y;
        nw[2] = q.nib.z;
        nw[3] = q.nib.w;
    }
    const h16x2 s16 = {(h16)0.0625f, (h16)0.0625f};
    if constexpr (T == AESIR_GGML_Q4_0) {
        const h16 d = bits_to_h((uint16_t)(q.s0 & 0xffffu));
        const h16x2 dd = {d, d};
        const h16x2 blo = {(h16)-1032.0f, (h16)-1032.0f}, bhi = {(h16)-72.0f, (h16)-72.0f};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const unsigned v = nw[j], t = v >> 8;
            a[j].x = h2_bits(q4_0_w2(as_h2((v & k.lo) | k.magic) + blo, dd));
            a[j].y = h2_bits(q4_0_w2(as_h2((t & k.lo) | k.magic) + blo, dd));
            a[j].z = h2_bits(q4_0_w2(__builtin_elementwise_fma(as_h2((v & k.hi) | k.magic), s16, bhi), dd));
            a[j].w = h2_bits(q4_0_w2(__builtin_elementwise_fma(as_h2((t & k.hi) | k.magic), s16, bhi), dd));
        }
    } else if constexpr (T == AESIR_GGML_Q2_K || T == AESIR_GGML_Q3_K) {
        // a scale per record (16 weights): the lane's two records have their own; the values are
        // q (Q2_K) or q - 4 (Q3_K, its nibble holding q + 4), then Q4_K's or Q6_K's rule
        constexpr float off = T == AESIR_GGML_Q3_K ? 4.0f : 0.0f;
        const h16x2 blo = {(h16)(-1024.0f - off), (h16)(-1024.0f - off)}, bhi = {(h16)(-64.0f - off), (h16)(-64.0f - off)};
        h16x2 aa[2], nbb[2];
        if constexpr (T == AESIR_GGML_Q2_K) {
            const h16x2 b1024 = {(h16)-1024.0f, (h16)-1024.0f};
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const unsigned x = q.s0 >> (8 * r);  // scale | min << 4
                const h16x2 sm = as_h2(((x & 15u) | ((x & 0xF0u) << 12)) | k.magic) + b1024;
                const h16x2 ab = q4k_scales(as_h2(q.s1), sm);
                aa[r] = h16x2{ab.x, ab.x};
                nbb[r] = h16x2{-ab.y, -ab.y};
            }
        } else {
            const h16x2 b1152 = {(h16)-1152.0f, (h16)-1152.0f};
            const h16x2 sc = as_h2(__builtin_amdgcn_perm(0u, q.s0 ^ 0x8080u, 0x0c010c00u) | k.magic) + b1152;
            const h16 d = bits_to_h((uint16_t)(q.s1 & 0xffffu));
            const h16x2 a01 = h16x2{d, d} * sc;  // (f16(d sc0), f16(d sc1))
            aa[0] = h16x2{a01.x, a01.x};
            aa[1] = h16x2{a01.y, a01.y};
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = j >> 1;
            auto rule = [&](h16x2 v) {
                if constexpr (T == AESIR_GGML_Q2_K) return q4k_w2(v, aa[r], nbb[r]);
                else return q6k_w2(v, aa[r]);
            };
            const unsigned v = nw[j], t = v >> 8;
            a[j].x = h2_bits(rule(as_h2((v & k.lo) | k.magic) + blo));
            a[j].y = h2_bits(rule(as_h2((t & k.lo) | k.magic) + blo));
            a[j].z = h2_bits(rule(__builtin_elementwise_fma(as_h2((v & k.hi) | k.magic), s16, bhi)));
            a[j].w = h2_bits(rule(__builtin_elementwise_fma(as_h2((t & k.hi) | k.magic), s16, bhi)));
        }
    } else if constexpr (T != AESIR_GGML_Q6_K) {
        // Q4_1, Q5_0, Q5_1, Q4_K, Q5_K: the exact quantized pairs (q - 16 for Q5_0, else q), the
        // fifth bits OR-ed in at value 16 (low nibbles) or 256 (16-scaled high nibbles), then the
        // weight rule with the record pair's scales
        constexpr bool h5 = qf_hb5<T>();
        constexpr float off = T == AESIR_GGML_Q5_0 ? 16.0f : 0.0f;
        const h16x2 blo = {(h16)(-1024.0f - off), (h16)(-1024.0f - off)}, bhi = {(h16)(-64.0f - off), (h16)(-64.0f - off)};
        h16x2 aa, nbb;
        if constexpr (qf_kq<T>()) {
            const h16x2 b1024 = {(h16)-1024.0f, (h16)-1024.0f};
            // (scale, min) bytes into the low byte of each half, then exact through the 1024 exponent
            const h16x2 sm = as_h2(__builtin_amdgcn_perm(0u, q.s0, 0x0c010c00u) | k.magic) + b1024;
            const h16x2 ab = q4k_scales(as_h2(q.s1), sm);
            aa = h16x2{ab.x, ab.x};
            nbb = h16x2{-ab.y, -ab.y};
        } else if constexpr (qf_dm<T>()) {
            const h16x2 dm = as_h2(q.s0);
            aa = h16x2{dm.x, dm.x};
            nbb = h16x2{dm.y, dm.y};
        } else {
            const h16 d = bits_to_h((uint16_t)(q.s0 & 0xffffu));
            aa = h16x2{d, d};
        }
        auto rule = [&](h16x2 v) {
            if constexpr (qf_kq<T>()) return q4k_w2(v, aa, nbb);
            else if constexpr (qf_dm<T>()) return q4_1_w2(v, aa, nbb);
            else return q4_0_w2(v, aa);
        };
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const unsigned v = nw[j], t = v >> 8;
            unsigned fa = 0u, fb = 0u, ga = 0u, gb = 0u;  // fifth bits of the four pairs
            if constexpr (h5) {
                const unsigned h = (j >> 1) ? q.hb >> 1 : q.hb;  // the record's bits at the even positions
                const unsigned ha = (j & 1) == 0 ? h << 4 : h >> 4, hb = (j & 1) == 0 ? h << 2 : h >> 6;
                fa = ha & k.flo;
                ga = ha & k.fhi;
                fb = hb & k.flo;
                gb = hb & k.fhi;
            }
            a[j].x = h2_bits(rule(as_h2(fa | ((v & k.lo) | k.magic)) + blo));
            a[j].y = h2_bits(rule(as_h2(fb | ((t & k.lo) | k.magic)) + blo));
            a[j].z = h2_bits(rule(__builtin_elementwise_fma(as_h2(ga | ((v & k.hi) | k.magic)), s16, bhi)));
            a[j].w = h2_bits(rule(__builtin_elementwise_fma(as_h2(gb | ((t & k.hi) | k.magic)), s16, bhi)));
        }
    } else {
        const h16x2 blo = {(h16)-1056.0f, (h16)-1056.0f}, bhi = {(h16)-96.0f, (h16)-96.0f};
        const h16x2 b1152 = {(h16)-1152.0f, (h16)-1152.0f};
        // int8 scales of the two records: byte ^ 0x80 under the 1024 exponent reads 1152 + sc
        const h16x2 sc = as_h2(__builtin_amdgcn_perm(0u, q.s0 ^ 0x8080u, 0x0c010c00u) | k.magic) + b1152;
        const h16 d = bits_to_h((uint16_t)(q.s1 & 0xffffu));
        const h16x2 a01 = h16x2{d, d} * sc;  // (f16(d sc0), f16(d sc1))
        const unsigned hw[2] = {q.hb.x, q.hb.y};
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const h16x2 aa = r == 0 ? h16x2{a01.x, a01.x} : h16x2{a01.y, a01.y};
            const unsigned h = hw[r];
#pragma unroll
            for (int wd = 0; wd < 2; wd++) {
                const int j = 2 * r + wd;
                const unsigned v = nw[j], t = v >> 8;
                const unsigned ha = wd == 0 ? h << 4 : h >> 4, hb = wd == 0 ? h << 2 : h >> 6;
                a[j].x = h2_bits(q6k_w2(as_h2((ha & k.hlo) | ((v & k.lo) | k.magic)) + blo, aa));
                a[j].y = h2_bits(q6k_w2(as_h2((hb & k.hlo) | ((t & k.lo) | k.magic)) + blo, aa));
                a[j].z = h2_bits(q6k_w2(__builtin_elementwise_fma(as_h2((ha & k.hhi) | ((v & k.hi) | k.magic)), s16, bhi), aa));
                a[j].w = h2_bits(q6k_w2(__builtin_elementwise_fma(as_h2((hb & k.hhi) | ((t & k.hi) | k.magic)), s16, bhi), aa));
            }
        }
    }
}

// x of one record (natural order, x[0]: elements 0..7, x[1]: 8..15) -> the B operands of its two
// nibble words: o[0] = elements {0, 2, 1, 3, 8, 10, 9, 11}, o[1] = the same + 4.
__device__ __forceinline__ void qf_perm_rec(const u32x4 (&x)[2], u32x4 (&o)[2]) {
    const unsigned e[8] = {x[0].x, x[0].y, x[0].z, x[0].w, x[1].x, x[1].y, x[1].z, x[1].w};
#pragma unroll
    for (int c = 0; c < 2; c++) {
        o[c].x = __builtin_amdgcn_perm(e[2 * c + 1], e[2 * c], 0x05040100u);
        o[c].y = __builtin_amdgcn_perm(e[2 * c + 1], e[2 * c], 0x07060302u);
        o[c].z = __builtin_amdgcn_perm(e[2 * c + 5], e[2 * c + 4], 0x05040100u);
        o[c].w = __builtin_amdgcn_perm(e[2 * c + 5], e[2 * c + 4], 0x07060302u);
    }
}

// x source: x itself, or (layer 0) row token->token of the repacked embedding table, dequantized
// in the workgroup, with workgroup 0 writing the row to xcopy (the residual stream).
struct QFXSrc {
    const h16 *x;
    QFMat emb;
    const DecodeState *token;
    h16 *xcopy;
};

// x records per thread held in registers while the first tiles load (larger K stages x in a loop
// after the tile requests).
constexpr int kQfXRegs = 1;

// The body of the decode GEMV for workgroup bid of nbid working on w's N rows; the epilogue sees
// row r of w as output row rbase + r of Nall (a matrix may be the second part of a fused one).
template <int T, int NW, int SP, int QD, bool NORM, class Epi>
__device__ __forceinline__ void gemv_qf_body(uint8_t *lds, const QFMat &w, int64_t N, int64_t K, const QFXSrc &src,
                                             const h16 *__restrict__ nw, float eps, const Epi &epi, int bid, int nbid,
                                             int64_t rbase, int64_t Nall) {
    constexpr int NT = NW * kWave, XR = kQfXRegs;
    // the lm_head keeps one argmax partial per 8 logits: its epilogue runs per 8 rows
    constexpr int ER = std::is_same<Epi, EpiLmHead>::value ? 8 : 16;
    static_assert(NW >= 16 / ER, "one epilogue wave per row group");
    // lds: x (2 K bytes), the row partials (2 x NW x 16), the norm scratch
    float *red = reinterpret_cast<float *>(lds + 2 * K);
    float *nred = red + 2 * NW * 16;  // NW floats, then 16 for the final row sums
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nseg = (int)(K / kSeg), nrec = (int)(K / kRec);
    const int blocks = (int)((N + 15) / 16);
    const int pb0 = (int)(w.row0 / 16);  // plane row block of row 0
    const QfRsrc rs = qf_rsrc(w, T, w.row0 + (int64_t)blocks * 16, K);
    constexpr int es1 = (qf_kq<T>() || T == AESIR_GGML_Q2_K) ? 4 : 2;
    const int sbr = (int)(K / 256);  // s1 entries per row
    const int s1v = (lane & 15) * es1;
    // steps of this workgroup: (block k, round r), r < R, for its nb blocks
    const int R = (nseg + NW * SP - 1) / (NW * SP);
    const int nb = (blocks - bid + nbid - 1) / nbid;
    const int steps = nb * R;
    if (nb <= 0) return;  // a grid larger than the blocks (never launched so)

    // x: record r of x itself, or of row token->token of the embedding table (dequantized)
    const bool embed = src.emb.nib != nullptr;
    const int64_t erow = embed ? src.emb.row0 + src.token->token : 0;
    h16 *xcopy = (src.xcopy && bid == 0) ? src.xcopy : nullptr;
    auto getx = [&](int r, u32x4(&x)[2]) {
        if (embed) {
            qf_deq16<T>(qf_load<T>(src.emb, erow, r, K), x);
        } else {
            x[0] = ld16(src.x + (int64_t)r * kRec);
            x[1] = ld16(src.x + (int64_t)r * kRec + 8);
        }
    };
    // Every load below is issued on all paths (a surplus thread or slot re-reads a valid, cached
    // address): the waits the compiler places before each use then count only the loads issued
    // after it, so the next round's tiles stay in flight while the current one computes.
    const bool xfast = nrec <= XR * NT;
    u32x4 xr[XR][2], nr[XR][2];
    if (xfast) {
#pragma unroll
        for (int j = 0; j < XR; j++) {
            const int r = tid + NT * j < nrec ? tid + NT * j : nrec - 1;
            getx(r, xr[j]);
            if (NORM) {
                nr[j][0] = ld16(nw + (int64_t)r * kRec);
                nr[j][1] = ld16(nw + (int64_t)r * kRec + 8);
            }
        }
    }

    // QD steps in flight: step st + QD - 1 is requested when step st starts (steps past the last
    // re-read the last step's tiles, so every path issues the same loads)
    QTile<T> tl[QD][SP];
    // the next step to request: its index, block ik and round ir, counted up step by step (no
    // division in the loop); past the last step the last one is requested again
    int ist = 0, ik = 0, ir = 0;
    auto issue_next = [&](QTile<T>(&buf)[SP]) {
        const bool live = ist < steps;
        const int kk = live ? ik : nb - 1, rr = live ? ir : R - 1;
        const int pb = pb0 + bid + kk * nbid, first = wave + NW * SP * rr;
#pragma unroll
        for (int i = 0; i < SP; i++) {
            const int sg = first + NW * i < nseg ? first + NW * i : nseg - 1;  // a surplus slot: the last segment
            buf[i] = qf_tile_load<T>(rs, pb * nseg + sg, lane, s1v, (pb * sbr + (int)((unsigned)sg >> 1)) * 16 * es1);
        }
        ++ist;
        if (++ir == R) {
            ir = 0;
            ++ik;
        }
    };
#pragma unroll
    for (int j = 0; j + 1 < QD; j++) issue_next(tl[j]);
    // the epilogue operands of this wave's rows (ER rows at en(k)) of the current and next block
    const bool ewave = wave < 16 / ER;
    auto en = [&](int k) { return rbase + (int64_t)(bid + k * nbid) * 16 + wave * ER; };
    using Pre = decltype(epi.template prefetch<ER>(0, 0, Nall, 0));
    Pre pre = epi.template prefetch<ER>(en(0), 0, Nall, ewave ? lane : kWave);

    // stage x: record r at lds + 32 r in the B-operand order, RMS-normalized when NORM
    h16 inv = (h16)1.0f;
    if (xfast) {
        if (NORM) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < XR; j++)
                if (tid + NT * j < nrec) ss = sumsq8(xr[j][1], sumsq8(xr[j][0], ss));
            ss = block_sum<NW, false>(ss, nred);
            inv = (h16)(1.0f / sqrtf(ss / (float)K + eps));
        }
#pragma unroll
        for (int j = 0; j < XR; j++) {
            const int r = tid + NT * j;
            if (r < nrec) {
                u32x4 o[2];
                if (xcopy) {
                    st16(xcopy + (int64_t)r * kRec, xr[j][0]);
                    st16(xcopy + (int64_t)r * kRec + 8, xr[j][1]);
                }
                if (NORM) {
                    xr[j][0] = norm8(xr[j][0], nr[j][0], inv);
                    xr[j][1] = norm8(xr[j][1], nr[j][1], inv);
                }
                qf_perm_rec(xr[j], o);
                st16(lds + 32 * r, o[0]);
                st16(lds + 32 * r + 16, o[1]);
            }
        }
    } else {
        if (NORM) {
            float ss = 0.0f;
            for (int r = tid; r < nrec; r += NT) {
                u32x4 x[2];
                getx(r, x);
                ss = sumsq8(x[1], sumsq8(x[0], ss));
            }
            ss = block_sum<NW, false>(ss, nred);
            inv = (h16)(1.0f / sqrtf(ss / (float)K + eps));
        }
        for (int r = tid; r < nrec; r += NT) {
            u32x4 x[2], o[2];
            getx(r, x);
            if (xcopy) {
                st16(xcopy + (int64_t)r * kRec, x[0]);
                st16(xcopy + (int64_t)r * kRec + 8, x[1]);
            }
            if (NORM) {
                x[0] = norm8(x[0], ld16(nw + (int64_t)r * kRec), inv);
                x[1] = norm8(x[1], ld16(nw + (int64_t)r * kRec + 8), inv);
            }
            qf_perm_rec(x, o);
            st16(lds + 32 * r, o[0]);
            st16(lds + 32 * r + 16, o[1]);
        }
    }
    __syncthreads();

    const QfRegs kr = QfRegs::make();
    f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
    float *fin = nred + NW;  // the block's final row sums, each ER-row part written and read by its epilogue wave
    // a step: request the step QD - 1 ahead into nxt, multiply the tiles of cur, and after a block's
    // last round reduce its row sums over the waves and run its epilogue
    int ck = 0, cr = 0;  // block and round of the current step
    auto step = [&](const QTile<T>(&cur)[SP], QTile<T>(&nxt)[SP]) {
        const int k = ck, r = cr;
        if (++cr == R) {
            cr = 0;
            ++ck;
        }
        issue_next(nxt);
        const int first = wave + NW * SP * r;
#pragma unroll
        for (int i = 0; i < SP; i++) {
            const int sg = first + NW * i;
            if (sg < nseg) {
                const uint8_t *xs = lds + sg * 256 + (lane >> 4) * 64;  // records 8 sg + 2 (lane / 16), + 1
                const u32x4 bx[4] = {ld16(xs), ld16(xs + 16), ld16(xs + 32), ld16(xs + 48)};
                u32x4 a[4];
                qf_tile_a<T>(cur[i], kr, a);
#pragma unroll
                for (int j = 0; j < 4; j++) acc[j & 1] = mfma16x16x32(a[j], bx[j], acc[j & 1]);
            }
        }
        if (r == R - 1) {
            float *rb = red + (k & 1) * (NW * 16);
            if ((lane & 15) == 0) {  // rows 4 (lane / 16) + e, the same in every column
                const f32x4 v = acc[0] + acc[1];
#pragma unroll
                for (int e = 0; e < 4; e++) rb[wave * 16 + 4 * (lane >> 4) + e] = v[e];
            }
            acc[0] = acc[1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            __syncthreads();
            const Pre now = pre;
            if (k + 1 < nb) pre = epi.template prefetch<ER>(en(k + 1), 0, Nall, ewave ? lane : kWave);
            if (ewave) {
                if (lane < ER) {  // lane: row wave * ER + lane, summed over the waves in one order
                    float v = rb[wave * ER + lane];
#pragma unroll
                    for (int w2 = 1; w2 < NW; w2++) v += rb[w2 * 16 + wave * ER + lane];
                    fin[wave * ER + lane] = v;
                }
                epi.template apply<ER>(en(k), 0, Nall, fin + wave * ER, lane, now);
            }
        }
    };
    // unrolled QD times so that every buffer keeps its registers
    for (int base = 0; base < steps; base += QD) {
#pragma unroll
        for (int j = 0; j < QD; j++)
            if (base + j < steps) step(tl[j], tl[(j + QD - 1) % QD]);
    }
}

template <int T, int NW, int SP, int QD, bool NORM, class Epi>
__global__ __launch_bounds__(NW * kWave) void gemv_qf_kernel(QFMat w, int64_t N, int64_t K, QFXSrc src,
                                                             const h16 *__restrict__ nw, float eps, Epi epi) {
    extern __shared__ __align__(16) uint8_t lds[];
    gemv_qf_body<T, NW, SP, QD, NORM, Epi>(lds, w, N, K, src, nw, eps, epi, (int)blockIdx.x, (int)gridDim.x, 0, N);
}

// One launch over a fused matrix stored in two parts of different types (a mixed Q/K/V): the
// first ga workgroups run part A's na rows (type TA), the others part B's nb rows (type TB) as
// output rows na .. na + nb - 1. Each workgroup keeps one type for its life, so the branch is
// uniform and both parts stream at once without a second launch's fixed cost.
template <int TA, int TB, int NW, int SPA, int SPB, int QD, bool NORM, class Epi>
__global__ __launch_bounds__(NW * kWave) void gemv_qf2_kernel(QFMat wa, int64_t na, int ga, QFMat wb, int64_t nb,
                                                              int64_t K, QFXSrc src, const h16 *__restrict__ nw,
                                                              float eps, Epi epi) {
    extern __shared__ __align__(16) uint8_t lds[];
    if ((int)blockIdx.x < ga)
        gemv_qf_body<TA, NW, SPA, QD, NORM, Epi>(lds, wa, na, K, src, nw, eps, epi, (int)blockIdx.x, ga, 0, na + nb);
    else
        gemv_qf_body<TB, NW, SPB, QD, NORM, Epi>(lds, wb, nb, K, src, nw, eps, epi, (int)blockIdx.x - ga,
                                                 (int)gridDim.x - ga, na, na + nb);
}

// Waves, round length and workgroups (measured on MI355X over the Llama-3-8B shapes): 8 waves with
// rounds of half the register budget's tiles; from 1024 blocks on, persistent workgroups (512,
// or 1024 from 4096 blocks, i.e. 3.5 to 8 blocks each), otherwise one block per workgroup.
// Steps (rounds of SP tiles) in flight per wave of the decode GEMV. Measured on MI355X
// (Llama-3-8B shape decode, KV 2048): 2 steps beat 3 and 4 for every type (Q4_0 657 / 621 / 586
// tok/s, Q4_K 617 / 582 / 551, Q6_K 520 / 496 / 479; gate/up 14.9 / 15.5 / 17.0 us for Q4_0).
constexpr int kQfDepth = 2;
struct QfShape {
    int nw, sp;
    int64_t grid;
};
static QfShape qf_shape(int64_t blocks, int round) {
    const int64_t grid = blocks < 1024 ? blocks : blocks < 4096 ? 512 : 1024;
    return {8, round / 2, grid};
}

template <bool NORM, class Epi, int T>
static void gemv_qf_launch_t(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const QFXSrc &src, const void *nwt,
                             float eps, const Epi &epi) {
    constexpr int RD = qf_round<T>();
    const QfShape sh = qf_shape((N + 15) / 16, RD);
    const size_t lds = (size_t)(2 * K) + ((size_t)sh.nw * (2 * 16 + 1) + 16) * sizeof(float);
    // Q6_K rows of at least 8192 weights (the down projection: few row blocks, one per workgroup,
    // each a long sequence of rounds) take rounds of 2 tiles, as the other types; shorter ones keep
    // 1. Measured at the Llama-3-8B shape in alternating runs: down 12.2-12.5 -> 11.8-12.1 us with 2
    // tiles, while gate/up (21.6-22.2 -> 21.6-23.3 us) and lm_head (75-76 -> 76-80 us) lose.
    if constexpr (T == AESIR_GGML_Q6_K) {
        if (K >= 8192) {
            hipLaunchKernelGGL((gemv_qf_kernel<T, 8, 2, kQfDepth, NORM, Epi>), dim3((unsigned)sh.grid), dim3(8 * kWave),
                               lds, s, w, N, K, src, (const h16 *)nwt, eps, epi);
            return;
        }
    }
    hipLaunchKernelGGL((gemv_qf_kernel<T, 8, RD / 2, kQfDepth, NORM, Epi>), dim3((unsigned)sh.grid), dim3(8 * kWave), lds, s,
                       w, N, K, src, (const h16 *)nwt, eps, epi);
}

bool qf_gemv_ok(int64_t K) { return K > 0 && K % kSeg == 0 && K <= kQfGemvMaxK; }

template <bool NORM, class Epi>
static int32_t gemv_qf_dispatch(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const QFXSrc &src, const void *nw,
                                float eps, const Epi &epi, const char *name) {
    AESIR_TRY(qf_check(w.type, K, name));
    if (!qf_gemv_ok(K))
        return fail(AESIR_ERR_UNSUPPORTED, "%s: quantized GEMV needs a row length that is a multiple of 128, at most %lld (got %lld)",
                    name, (long long)kQfGemvMaxK, (long long)K);
    if (w.row0 % 16 != 0) return fail(AESIR_ERR_INVALID, "%s: quantized GEMV needs a matrix starting on a 16-row block", name);
    if (src.emb.nib && src.emb.type != w.type) return fail(AESIR_ERR_INVALID, "%s: embedding type differs", name);
    const void *xp = src.emb.nib ? (const void *)src.emb.nib : (const void *)src.x;
    if (((uintptr_t)w.nib & 15) || ((uintptr_t)xp & 15) || (NORM && ((uintptr_t)nw & 15)) ||
        (src.xcopy && ((uintptr_t)src.xcopy & 15)))
        return fail(AESIR_ERR_UNSUPPORTED, "%s: quantized GEMV needs 16-byte aligned operands", name);
    if (N <= 0) return AESIR_OK;
    // plane offsets are 32-bit in the buffer loads
    if (mul_checked(w.row0 + qf_rows_alloc(N), qf_plane_row_bytes(w.type, 0, K)) > INT32_MAX)
        return fail(AESIR_ERR_UNSUPPORTED, "%s: matrix of %lld x %lld exceeds 2 GiB of 4-bit weights", name, (long long)N,
                    (long long)K);
    qf_switch(w.type, [&](auto t) { gemv_qf_launch_t<NORM, Epi, decltype(t)::value>(s, w, N, K, src, nw, eps, epi); });
    AESIR_LAUNCH_CHECK(name);
    return AESIR_OK;
}

int32_t launch_qf_gemv_store(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const void *x, void *y) {
    EpiStore e{(h16 *)y, N};
    return gemv_qf_dispatch<false>(s, w, N, K, QFXSrc{(const h16 *)x, QFMat{}, nullptr, nullptr}, nullptr, 0.0f, e,
                                   "gemv_qf_store");
}

int32_t launch_qf_gemv_residual(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const void *x_in, void *x) {
    EpiResidual e{(h16 *)x};
    return gemv_qf_dispatch<false>(s, w, N, K, QFXSrc{(const h16 *)x_in, QFMat{}, nullptr, nullptr}, nullptr, 0.0f, e,
                                   "gemv_qf_residual");
}

int32_t launch_qf_gate_up_swiglu(hipStream_t s, const void *x, const void *norm_w, float eps, const QFMat &w,
                                 int64_t ffn, int64_t dim, void *act) {
    EpiSwiglu e{(h16 *)act};
    return gemv_qf_dispatch<true>(s, w, 2 * ffn, dim, QFXSrc{(const h16 *)x, QFMat{}, nullptr, nullptr}, norm_w, eps, e,
                                  "gemv_qf_gate_up");
}

// Type pairs of a Q/K/V matrix stored in two parts (rows [0, split) of type A, the rest of type B),
// as the K-quant mixes lay out attn_q / attn_k and attn_v (a higher-bit V, or a higher-bit K and V).
template <class F>
static bool qf_pair_switch(int32_t ta, int32_t tb, F &&f) {
#define AESIR_QF_PAIR(A, B)                                                                          \
    if (ta == A && tb == B) {                                                                        \
        f(std::integral_constant<int, A>{}, std::integral_constant<int, B>{});                       \
        return true;                                                                                 \
    }
    AESIR_QF_PAIR(AESIR_GGML_Q4_K, AESIR_GGML_Q6_K)
    AESIR_QF_PAIR(AESIR_GGML_Q5_K, AESIR_GGML_Q6_K)
    AESIR_QF_PAIR(AESIR_GGML_Q4_K, AESIR_GGML_Q5_K)
    AESIR_QF_PAIR(AESIR_GGML_Q3_K, AESIR_GGML_Q4_K)
    AESIR_QF_PAIR(AESIR_GGML_Q3_K, AESIR_GGML_Q5_K)
    AESIR_QF_PAIR(AESIR_GGML_Q2_K, AESIR_GGML_Q4_K)
#undef AESIR_QF_PAIR
    return false;
}

bool qf_qkv_pair_ok(int32_t type_a, int32_t type_b) {
    return qf_pair_switch(type_a, type_b, [](auto, auto) {});
}

int32_t launch_qf_qkv_rope_kv(hipStream_t s, const QkvArgs &a, const EpiQkv &e) {
    const QFXSrc src = a.eq.nib ? QFXSrc{nullptr, a.eq, a.state, (h16 *)a.x}
                                : QFXSrc{(const h16 *)a.x, QFMat{}, nullptr, nullptr};
    const int64_t N = a.dim + 2 * a.kvd, K = a.dim;
    if (a.qkv_split <= 0)
        return gemv_qf_dispatch<true>(s, a.wq, N, K, src, a.norm_w, a.eps, e, "gemv_qf_qkv_rope_kv");
    // two parts: one launch, each workgroup on one part (the embedding lookup runs apart)
    const char *name = "gemv_qf2_qkv_rope_kv";
    const int64_t na = a.qkv_split, nb = N - na;
    if (na % 16 != 0 || nb <= 0 || a.eq.nib) return fail(AESIR_ERR_INVALID, "%s: bad part split", name);
    AESIR_TRY(qf_check(a.wq.type, K, name));
    AESIR_TRY(qf_check(a.wq_b.type, K, name));
    if (!qf_gemv_ok(K)) return fail(AESIR_ERR_UNSUPPORTED, "%s: row length %lld", name, (long long)K);
    if (((uintptr_t)a.wq.nib & 15) || ((uintptr_t)a.wq_b.nib & 15) || ((uintptr_t)a.x & 15) || ((uintptr_t)a.norm_w & 15))
        return fail(AESIR_ERR_UNSUPPORTED, "%s: quantized GEMV needs 16-byte aligned operands", name);
    bool launched = false;
    qf_pair_switch(a.wq.type, a.wq_b.type, [&](auto ta, auto tb) {
        constexpr int TA = decltype(ta)::value, TB = decltype(tb)::value;
        constexpr int RA = qf_round<TA>(), RB = qf_round<TB>();
        const QfShape sa = qf_shape((na + 15) / 16, RA), sb = qf_shape((nb + 15) / 16, RB);
        const size_t lds = (size_t)(2 * K) + ((size_t)8 * (2 * 16 + 1) + 16) * sizeof(float);
        hipLaunchKernelGGL((gemv_qf2_kernel<TA, TB, 8, RA / 2, RB / 2, kQfDepth, true, EpiQkv>),
                           dim3((unsigned)(sa.grid + sb.grid)), dim3(8 * kWave), lds, s, a.wq, na, (int)sa.grid, a.wq_b, nb,
                           K, src, (const h16 *)a.norm_w, a.eps, e);
        launched = true;
    });
    if (!launched)
        return fail(AESIR_ERR_UNSUPPORTED, "%s: no two-part GEMV for types %s and %s", name, ggml_type_name(a.wq.type),
                    ggml_type_name(a.wq_b.type));
    AESIR_LAUNCH_CHECK(name);
    return AESIR_OK;
}

int32_t launch_qf_lm_head(hipStream_t s, const LmHeadArgs &a, const EpiLmHead &e) {
    return gemv_qf_dispatch<true>(s, a.wq, a.vocab, a.dim, QFXSrc{(const h16 *)a.x, QFMat{}, nullptr, nullptr},
                                  a.norm_w, a.eps, e, "gemv_qf_lm_head");
}

// ------------------------------------------------------------------ batched-prefill GEMM

// C = epilogue(A W^T) for a chunk of up to 128 activation rows and a matrix in the tiled planes,
// on v_mfma_f32_16x16x32_f16 without an f16 copy of the weights. Grid (N / NT, ceil(M / 128),
// K splits); 8 waves as 4 x 2, each 32 rows x NT / 2 columns. Per 128-wide K chunk (one tile
// column of the planes) the 128 activation rows (256-byte row chunks, granule p of row r holding
// k-granule p ^ (r & 15)) and the NT / 16 weight tiles' plane bytes (nibbles 1 KiB, s0, hb and the
// tile rows' s1 entries, each a contiguous run copied as laid out in memory) go straight into
// an LDS stage by buffer loads with the LDS destination; 3 stages, two chunks in flight, explicit
// wait counts per wave. A wave turns its tiles into MFMA operands with qf_tile_a (the decode
// GEMV's dequantization, so the weights are the same f16 values) and its activation rows into
// the matching k order with qf_perm_rec. Split z writes f32 partials like the f16 kernels.
constexpr int kQgA = kWideMT * kWideKC * 2;  // activation bytes per stage
constexpr int kQgTile = 2048;                // LDS bytes per weight tile: nib 1024, s0 256, hb 512, s1 256
__host__ __device__ constexpr int qg_stage_bytes(int nt) { return kQgA + nt / 16 * kQgTile; }
template <int T>
constexpr bool qg_has_s1() {
    return qf_kq<T>() || T == AESIR_GGML_Q2_K || T == AESIR_GGML_Q3_K || T == AESIR_GGML_Q6_K;
}
template <int T>
constexpr int qg_hb_copies() {
    return T == AESIR_GGML_Q6_K ? 2 : qf_hb5<T>() ? 1 : 0;
}
template <int T>
constexpr int qg_tile_copies() {
    return 2 + qg_hb_copies<T>() + (qg_has_s1<T>() ? 1 : 0);
}

template <int EPI, int NT, int T>
__global__ __launch_bounds__(kWideThreads) void gemm_wide_qf_kernel(const h16 *__restrict__ A, int64_t M, int64_t K,
                                                                   QFMat w, int64_t N, h16 *__restrict__ C,
                                                                   int64_t ldc, float *__restrict__ P) {
    constexpr int NTT = NT / 16;                         // weight tiles per workgroup
    constexpr int NCP = qg_tile_copies<T>(), NB = NTT * NCP;  // copies per tile and per chunk
    constexpr int NBW = (NB + 7) / 8, NBX = NB % 8;      // per wave: NBW copies below wave NBX, else NB / 8
    constexpr int kStage = qg_stage_bytes(NT);
    constexpr int MF = 2, NF = NT / 32;
    constexpr bool dm = qf_dm<T>();
    constexpr int s0b = dm ? 4 : 2;                      // s0 bytes per lane
    constexpr int es1 = (qf_kq<T>() || T == AESIR_GGML_Q2_K) ? 4 : 2;
    static_assert(NT == 32 || NT == 64, "tile width");
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / 2, wn = wave % 2;
    const int64_t m0 = (int64_t)blockIdx.y * kWideMT, n0 = (int64_t)blockIdx.x * NT;
    const int r = lane & 15, g = lane >> 4;
    const int nseg = (int)(K / kSeg), sbr = (int)(K / 256), pb0 = (int)(n0 / 16);
    const int64_t splits = gridDim.z, z = blockIdx.z;
    const int64_t c0 = nseg * z / splits, c1 = nseg * (z + 1) / splits;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void *)A, 0, (int)(M * K * 2), kBufferDword3);
    const QfRsrc rs = qf_rsrc(w, T, qf_rows_alloc(N), K);
    // activation copy j of this wave: rows 16 wave + 4 j .. + 3, lane l row + l / 16, granule l % 16
    int aoff[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int row = 16 * wave + 4 * j + (lane >> 4);
        aoff[j] = (int)((m0 + row) * K * 2) + (((lane & 15) ^ (row & 15)) << 4);
    }
    const int nbw = NBX == 0 || wave < NBX ? NBW : NBW - 1;  // this wave's weight copies per chunk
    auto issue = [&](int64_t c, int stage) {
        c = c < c1 ? c : c1 - 1;  // past the split's end: re-read its last chunk into a free stage
        uint8_t *sa = lds + stage * kStage;
#pragma unroll
        for (int j = 0; j < 4; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void *)(sa + (16 * wave + 4 * j) * (kWideKC * 2)), 16, aoff[j],
                (int)(c * kWideKC * 2), 0, 0);
        uint8_t *sb = sa + kQgA;
#pragma unroll
        for (int jb = 0; jb < NBW; jb++) {
            const int b = wave + 8 * jb;  // wave-uniform
            if (b >= NB) break;
            const int tb = b / NCP, kind = b % NCP, pb = pb0 + tb, pt = pb * nseg + (int)c;
            uint8_t *dst = sb + tb * kQgTile;
            constexpr int QB = 64 * qf_lane_bytes(T);  // quant-plane bytes per tile: 1024, 512 or 768
            if (kind == 0) {  // 16 bytes per lane, the first QB / 16 lanes
                if (QB == 1024 || lane < QB / 16)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs.nib, (__attribute__((address_space(3))) void *)dst, 16,
                                                             lane * 16, pt * QB, 0, 0);
            } else if (kind == 1) {  // 256 bytes from the tile's s0 (128 of them used with 2 bytes per lane)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs.s0, (__attribute__((address_space(3))) void *)(dst + 1024),
                                                         4, lane * 4, pt * 64 * s0b, 0, 0);
            } else if (kind < 2 + qg_hb_copies<T>()) {
                const int h = kind - 2;  // Q6_K: two 256-byte halves of the tile's 512
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rs.hb, (__attribute__((address_space(3))) void *)(dst + 1280 + 256 * h), 4, lane * 4,
                    pt * 256 * qg_hb_copies<T>() + 256 * h, 0, 0);
            } else {  // the row block's s1 entries of the chunk's super-block (and what follows)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs.s1, (__attribute__((address_space(3))) void *)(dst + 1792), 4,
                                                         lane * 4, (pb * sbr + (int)(c / 2)) * 16 * es1, 0, 0);
            }
        }
    };
    // wait until only the next chunk's copies are in flight (wave-uniform count)
    auto wait_chunk = [&]() {
        if (nbw == NBW) __builtin_amdgcn_s_waitcnt(vm_wait((4 + NBW) * (kWideS - 2)));
        else __builtin_amdgcn_s_waitcnt(vm_wait((4 + NBW - 1) * (kWideS - 2)));
    };
    const QfRegs kr = QfRegs::make();
    f32x4 acc[MF][NF];
#pragma unroll
    for (int i = 0; i < MF; i++)
#pragma unroll
        for (int f = 0; f < NF; f++) acc[i][f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < kWideS - 1; j++) issue(c0 + j, j);
    for (int64_t c = c0; c < c1; c++) {
        const int t = (int)((c - c0) % kWideS);
        wait_chunk();                                      // this wave's copies of chunk c ...
        __builtin_amdgcn_s_barrier();                      // ... and every wave's
        issue(c + kWideS - 1, (t + kWideS - 1) % kWideS);  // into the stage chunk c - 1 used
        const uint8_t *sa = lds + t * kStage, *sb = sa + kQgA;
        u32x4 ao[MF][4], bo[NF][4];
#pragma unroll
        for (int i = 0; i < MF; i++) {
            const int row = 32 * wm + 16 * i + r;
#pragma unroll
            for (int h = 0; h < 2; h++) {  // record 2 g + h of the row's chunk: k-granules 4 g + 2 h, + 1
                const u32x4 x[2] = {ld16(sa + row * (kWideKC * 2) + (((4 * g + 2 * h) ^ (row & 15)) << 4)),
                                    ld16(sa + row * (kWideKC * 2) + (((4 * g + 2 * h + 1) ^ (row & 15)) << 4))};
                u32x4 o[2];
                qf_perm_rec(x, o);
                ao[i][2 * h] = o[0];
                ao[i][2 * h + 1] = o[1];
            }
        }
#pragma unroll
        for (int f = 0; f < NF; f++) {
            const uint8_t *tp = sb + (wn * NF + f) * kQgTile;
            QTile<T> q;
            if constexpr (T == AESIR_GGML_Q2_K) {
                q.cr = *reinterpret_cast<const u32x2 *>(tp + lane * 8);
            } else if constexpr (T == AESIR_GGML_Q3_K) {
                const unsigned *pq = reinterpret_cast<const unsigned *>(tp + lane * 12);
                q.cr = u32x2{pq[0], pq[1]};
                q.hb = pq[2];
            } else {
                q.nib = ld16(tp + lane * 16);
            }
            if constexpr (dm) q.s0 = *reinterpret_cast<const unsigned *>(tp + 1024 + lane * 4);
            else q.s0 = *reinterpret_cast<const uint16_t *>(tp + 1024 + lane * 2);
            if constexpr (qf_hb5<T>()) q.hb = *reinterpret_cast<const unsigned *>(tp + 1280 + lane * 4);
            if constexpr (T == AESIR_GGML_Q6_K) q.hb = *reinterpret_cast<const u32x2 *>(tp + 1280 + lane * 8);
            if constexpr (es1 == 4 && qg_has_s1<T>()) q.s1 = *reinterpret_cast<const unsigned *>(tp + 1792 + r * 4);
            if constexpr (es1 == 2 && qg_has_s1<T>()) q.s1 = *reinterpret_cast<const uint16_t *>(tp + 1792 + r * 2);
            qf_tile_a<T>(q, kr, bo[f]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int i = 0; i < MF; i++)
#pragma unroll
                for (int f = 0; f < NF; f++) acc[i][f] = mfma16x16x32(ao[i][j], bo[f][j], acc[i][f]);
        __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(0));  // no copy may land in LDS after the workgroup ends
#pragma unroll
    for (int i = 0; i < MF; i++)
#pragma unroll
        for (int f = 0; f < NF; f++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int64_t m = m0 + 32 * wm + 16 * i + 4 * g + e;
                const int64_t n = n0 + wn * (NT / 2) + 16 * f + r;
                const float v = acc[i][f][e];
                if (splits == 1) {
                    const float partner = dpp_f<kDppXor1>(v);  // lane r ^ 1 holds column n ^ 1
                    gemm_epilogue<EPI>(C, ldc, M, N, m, n, v, partner);
                } else if (m < M && n < N) {
                    P[(z * M + m) * N + n] = v;
                }
            }
}

template <int EPI, int NT, int T>
static int32_t launch_qf_wide(hipStream_t s, const void *A, int64_t M, int64_t K, const QFMat &w, int64_t N, void *C,
                              int64_t ldc, float *part, int64_t splits) {
    static std::atomic<uint64_t> lds_set{0};
    constexpr int lds = kWideS * qg_stage_bytes(NT);
    AESIR_TRY(raise_lds_limit(reinterpret_cast<const void *>(gemm_wide_qf_kernel<EPI, NT, T>), lds, lds_set));
    const dim3 grid((unsigned)((N + NT - 1) / NT), (unsigned)((M + kWideMT - 1) / kWideMT), (unsigned)splits);
    hipLaunchKernelGGL((gemm_wide_qf_kernel<EPI, NT, T>), grid, dim3(kWideThreads), lds, s, (const h16 *)A, M, K, w, N,
                       (h16 *)C, ldc, part);
    return AESIR_OK;
}

int32_t launch_qf_gemm_wide(hipStream_t s, int epi, int nt, const void *A, int64_t M, int64_t K, const QFMat &w,
                            int64_t N, void *C, int64_t ldc, float *part, int64_t splits) {
    if (!qf_type(w.type) || w.row0 != 0 || K % kSeg != 0 || (nt != 32 && nt != 64) || splits < 1 || M < 1 || N < 1 ||
        (epi == kEpiSwiglu && (N & 1)) || (splits > 1 && !part))
        return fail(AESIR_ERR_INVALID, "gemm_qf_wide: unsupported arguments");
    const int64_t lim = (int64_t)1 << 31;
    if ((M + kWideMT) * K * 2 >= lim || qf_rows_alloc(N) * K >= lim)
        return fail(AESIR_ERR_UNSUPPORTED, "gemm_qf_wide: operand exceeds a 32-bit byte range");
    int32_t rc = AESIR_OK;
    qf_switch(w.type, [&](auto t) {
        constexpr int T = decltype(t)::value;
#define AESIR_QG(E, NTV) rc = launch_qf_wide<E, NTV, T>(s, A, M, K, w, N, C, ldc, part, splits)
        if (epi == kEpiStore) { if (nt == 64) AESIR_QG(kEpiStore, 64); else AESIR_QG(kEpiStore, 32); }
        else if (epi == kEpiResidual) { if (nt == 64) AESIR_QG(kEpiResidual, 64); else AESIR_QG(kEpiResidual, 32); }
        else { if (nt == 64) AESIR_QG(kEpiSwiglu, 64); else AESIR_QG(kEpiSwiglu, 32); }
#undef AESIR_QG
    });
    AESIR_TRY(rc);
    AESIR_LAUNCH_CHECK("gemm_wide_qf_kernel");
    return AESIR_OK;
}

}  // namespace aesir
