// Launchers of the gfx950 kernels (host-callable), shared by the C-ABI wrappers and the model.
#pragma once

#include "common.hpp"

namespace aesir {

// Position state of one decode step, resident in device memory so that a captured HIP graph
// can be replayed for every step: kernels read token/pos from here, and the lm_head kernel
// writes the greedy token back (and, in autoregressive mode, advances token/pos).
struct DecodeState {
    int64_t token;       // token evaluated by this step
    int64_t pos;         // its position (start_pos)
    int64_t next_token;  // argmax written by the lm_head kernel
    int64_t step;        // autoregressive step counter (index into the token ring)
    int64_t advance;     // nonzero: lm_head sets token = next_token, pos += 1, step += 1
    int64_t ring_cap;    // capacity of the token ring
    int64_t pad[2];
};

// ------------------------------------------------------------------ GEMV / GEMM (gemv.hip)

// C[m, n] = f16(sum_k A[m,k] B[n,k]) for M rows of A (decode GEMV per row; f32 accumulation).
int32_t launch_gemm_f16(aesir_ctx *ctx, const void *A, int64_t M, int64_t K, const void *B, int64_t N, void *C);
// Batched-prefill GEMM on MFMA tiles (M > 1); falls back to the GEMV path for shapes it does
// not tile.
int32_t launch_gemm_f16_mfma(aesir_ctx *ctx, const void *A, int64_t M, int64_t K, const void *B, int64_t N,
                             void *C);

// A Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q4_K, Q5_K or Q6_K matrix [N][K] in HBM (quant.hip),
// repacked from its GGUF blocks into records of 16 weights: record r of a row holds weights
// 16 r .. 16 r + 15.
//   nib  8 bytes per record: byte j holds weight 16 r + j in its low nibble and 16 r + 8 + j in
//        its high nibble (Q5_*, Q6_K: the low 4 bits; Q2_K: the 2-bit value; Q3_K: the 3-bit
//        value q + 4, hmask bit included);
//   hb   Q6_K: 4 bytes per record, the high 2 bits of the record's weights; Q5_0 / Q5_1 / Q5_K:
//        4 bytes per record pair, the fifth bits of both records in one word (bit layout in
//        quant.hip, qf_hb_pos);
//   s0   Q4_0 / Q5_0: f16 d per 32 weights; Q4_1 / Q5_1: f16 d | f16 m << 16 per 32 weights;
//        Q4_K / Q5_K: (scale, min) bytes per 32 weights, 6-bit values unpacked; Q6_K / Q3_K: int8
//        scale per 16 weights; Q2_K: GGML's scale | min << 4 byte per 16 weights;
//   s1   Q2_K / Q4_K / Q5_K: (d, dmin) f16 pair per 256 weights; Q3_K / Q6_K: f16 d per 256 weights.
// The nib, hb and s0 planes are tiled for the matrix-core GEMV: rows in blocks of 16 and records
// in segments of 8 (128 weights, K a multiple of 128); tile (row block, segment) stores, for
// record pair q = (record % 8) / 2 and row i of the block, the pair's 16 nibble bytes (8 or 4 hb
// bytes, 2 or 4 s0 bytes) at [q][i], so that lane l of a wave reading that many bytes at l times
// that size gets row l % 16 and record pair l / 16: the A-operand layout of
// v_mfma_f32_16x16x32_f16. s1 is [row block][K / 256][row % 16] (the 16 rows' entries of a
// super-block together). Planes hold qf_rows_alloc(N) rows (whole row blocks). Logical row r of
// a fused sub-matrix is plane row row0 + r * step (step 2 for the interleaved gate/up rows).
struct QFMat {
    int32_t type = 0;
    const void *nib = nullptr, *hb = nullptr, *s0 = nullptr, *s1 = nullptr;
    int64_t row0 = 0;
};
// Bytes per lane (record pair) of a tile's quant plane: 16 nibble bytes, or for Q2_K the two
// records' 2-bit crumb words (8), for Q3_K those plus the pair's third-bit word (12).
__host__ __device__ constexpr int qf_lane_bytes(int32_t type) {
    return type == AESIR_GGML_Q2_K ? 8 : type == AESIR_GGML_Q3_K ? 12 : 16;
}
// hb bytes per record pair (0 without the plane) and s0 bytes per record pair.
__host__ __device__ inline int qf_hb_bytes(int32_t type) {
    return type == AESIR_GGML_Q6_K ? 8
           : (type == AESIR_GGML_Q5_0 || type == AESIR_GGML_Q5_1 || type == AESIR_GGML_Q5_K) ? 4
                                                                                            : 0;
}
__host__ __device__ inline int qf_s0_bytes(int32_t type) {
    return (type == AESIR_GGML_Q4_1 || type == AESIR_GGML_Q5_1) ? 4 : 2;
}
// Bytes of one row of each plane (0 if the type has no such plane). plane: 0 nib, 1 hb, 2 s0, 3 s1.
__host__ __device__ inline int64_t qf_plane_row_bytes(int32_t type, int plane, int64_t K) {
    switch (plane) {
        case 0: return K / 32 * qf_lane_bytes(type);
        case 1: return K / 32 * qf_hb_bytes(type);
        case 2: return K / 32 * qf_s0_bytes(type);
        case 3:
            return (type == AESIR_GGML_Q4_K || type == AESIR_GGML_Q5_K || type == AESIR_GGML_Q2_K) ? K / 256 * 4
                   : (type == AESIR_GGML_Q6_K || type == AESIR_GGML_Q3_K)                          ? K / 256 * 2
                                                                                                   : 0;
        default: return 0;
    }
}
// Plane rows allocated for an N-row matrix (whole 16-row blocks).
__host__ __device__ inline int64_t qf_rows_alloc(int64_t N) { return (N + 15) / 16 * 16; }
// Tile of (plane row r, record rec) and the byte offsets of the record's planes.
__host__ __device__ inline int64_t qf_tile(int64_t r, int64_t rec, int64_t K) { return (r >> 4) * (K >> 7) + (rec >> 3); }
// The quant-plane bytes of the record's pair: lane l of a wave reading lb bytes at lb l gets the
// pair of records 2 (l / 16), + 1 of row l % 16 in the tile (lb = qf_lane_bytes).
__host__ __device__ inline int64_t qf_qlane_off(int64_t r, int64_t rec, int64_t K, int lb) {
    return qf_tile(r, rec, K) * 64 * lb + (((rec & 7) >> 1) * 16 + (r & 15)) * lb;
}
__host__ __device__ inline int64_t qf_nib_off(int64_t r, int64_t rec, int64_t K) {
    return qf_qlane_off(r, rec, K, 16) + (rec & 1) * 8;
}
// hb entry of the record's pair (es = qf_hb_bytes); Q6_K's word of the record is at + 4 (rec & 1)
__host__ __device__ inline int64_t qf_hb_pair_off(int64_t r, int64_t rec, int64_t K, int es) {
    return qf_tile(r, rec, K) * 64 * es + ((rec & 7) >> 1) * 16 * es + (r & 15) * es;
}
__host__ __device__ inline int64_t qf_hbw_off(int64_t r, int64_t rec, int64_t K) {
    return qf_hb_pair_off(r, rec, K, 8) + (rec & 1) * 4;
}
// s0 entry of the record's pair (es = qf_s0_bytes: Q4_0 / Q5_0 d, Q4_1 / Q5_1 d | m << 16,
// Q4_K / Q5_K scale | min << 8); Q6_K's byte of the record is at + (rec & 1)
__host__ __device__ inline int64_t qf_s0_off(int64_t r, int64_t rec, int64_t K, int es = 2) {
    return qf_tile(r, rec, K) * 64 * es + ((rec & 7) >> 1) * 16 * es + (r & 15) * es;
}
__host__ __device__ inline int64_t qf_s1_off(int64_t r, int64_t rec, int64_t K, int esize) {
    return (((r >> 4) * (K >> 8) + (rec >> 4)) * 16 + (r & 15)) * esize;
}
// True for the types this layout serves.
bool qf_type(int32_t type);
// GGUF blocks (rows x K, packed, device memory) -> planes of rows dst.row0 + r * step.
int32_t launch_qf_repack(hipStream_t s, int32_t type, const void *blocks, int64_t rows, int64_t K, const QFMat &dst,
                         int64_t step);
// Planes -> f16 [rows][K] (out_stride elements per output row); `row_ids` (device, may be null)
// selects the source rows (embedding lookups), else rows 0 .. rows - 1 (of w.row0, `step` apart).
int32_t launch_qf_dequant(hipStream_t s, const QFMat &w, int64_t rows, int64_t K, int64_t step,
                          const int64_t *row_ids, void *out, int64_t out_stride);
// Seeded synthetic planes: weights of standard deviation near `std`, mean near 0.
int32_t launch_qf_fill_random(hipStream_t s, const QFMat &w, int64_t rows, int64_t K, int64_t step, uint64_t seed,
                              uint64_t stream, float std);
// GGUF blocks (rows x K, packed, device memory; Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q4_K,
// Q5_K or Q6_K) -> f16 rows of out_stride weights, straight from the blocks, the same f16 values
// as launch_qf_dequant and the Q8_0 GEMV (the per-op GEMMs of 16 or more rows, row lengths the
// GEMV does not take, the types without repacked planes, and the quantized parts of a model
// matrix stored in f16).
int32_t launch_gguf_dequant(hipStream_t s, int32_t type, const void *blocks, int64_t rows, int64_t K, void *out,
                            int64_t out_stride);
// Weights per block of a GGML block type launch_gguf_dequant takes (32 or 256), else 0.
int64_t gguf_block_elems(int32_t type);
// The decode GEMV stages x in LDS (2 K bytes) and works on whole 128-weight segments.
constexpr int64_t kQfGemvMaxK = 28672;
// The Q8_0 decode GEMV holds x in registers, 16 values per thread per 4096-wide slab, 7 slabs.
constexpr int64_t kQ8GemvMaxK = 28672;
bool qf_gemv_ok(int64_t K);
// Batched-prefill GEMM on a repacked matrix (row0 0, K % 128 == 0): C = epilogue epi (store /
// residual / SwiGLU, the GemmEpi values) of A [M][K] x W^T, nt = 64 or 32 columns per workgroup,
// `splits` K splits writing f32 partials to `part` ([splits][M][N]) when above 1.
int32_t launch_qf_gemm_wide(hipStream_t s, int epi, int nt, const void *A, int64_t M, int64_t K, const QFMat &w,
                            int64_t N, void *C, int64_t ldc, float *part, int64_t splits);
// Whether launch_gemm_qf_mfma takes an M x K by N x K product (more than 64 rows, K % 128 == 0,
// 32-bit byte ranges), and that product stored as f16 C [M][N] (context stream and partials).
bool gemm_qf_wide_ok(int64_t M, int64_t K, int64_t N);
int32_t launch_gemm_qf_mfma(aesir_ctx *ctx, const void *A, int64_t M, int64_t K, const QFMat &w, int64_t N, void *C);
// y[n] = f16(sum_k x[k] w[n, k]) for one row of x (the per-op GEMV of a repacked matrix).
int32_t launch_qf_gemv_store(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const void *x, void *y);
// Decode-step GEMVs of repacked matrices with the fused epilogues (see the F16 launchers).
int32_t launch_qf_gemv_residual(hipStream_t s, const QFMat &w, int64_t N, int64_t K, const void *x_in, void *x);
int32_t launch_qf_gate_up_swiglu(hipStream_t s, const void *x, const void *norm_w, float eps, const QFMat &w,
                                 int64_t ffn, int64_t dim, void *act);

// Fused decode-step GEMVs. All pointers are device pointers inside the model's arena.
struct QkvArgs {
    const void *x;          // residual stream [dim] (pre-norm)
    const void *embd;       // layer 0 only: token_embd [vocab][dim]; x = embd[state->token] is
                            // staged from it and copied to `x` (the embedding lookup, fused)
    const void *norm_w;     // attn_norm [dim]
    float eps;
    const void *w;          // [dim + 2*kvd][dim]: Q rows, K rows, V rows
    int64_t dim, kvd, head_dim;
    void *q_out;            // [dim]
    void *k_cache, *v_cache;  // this layer's [max_seq][kvd]
    int64_t max_seq;
    const void *rope;       // [n_pos][head_dim/2] (cos, sin) f16 pairs
    const DecodeState *state;
    const void *w_scale;    // Q8_0 weights: f16 block scales [dim + 2*kvd][dim / 32] (w is then int8);
                            // null for f16 weights
    const void *embd_scale; // layer 0 of a Q8_0 model: token_embd block scales (embd is then int8)
    QFMat wq;               // Q4_0 / Q4_K / Q6_K models: the QKV matrix (w and w_scale unused)
    QFMat eq;               // layer 0 of such a model: token_embd (embd unused)
    int64_t qkv_split = 0;  // > 0: wq holds rows [0, qkv_split), wq_b the rest, in another type
    QFMat wq_b;
};
int32_t launch_qkv_rope_kv(hipStream_t s, const QkvArgs &a);
// True when a Q/K/V matrix can be stored as two parts of these repacked types (rows of type_a,
// then rows of type_b) and run by one two-part GEMV launch.
bool qf_qkv_pair_ok(int32_t type_a, int32_t type_b);

// x[n] = f16(f16(W x_in)[n] + x[n]) (O projection and down projection with the residual add).
// w_scale non-null: W is Q8_0 (int8 quants [N][K] + f16 scales [N][K/32]).
int32_t launch_gemv_residual(hipStream_t s, const void *w, int64_t N, int64_t K, const void *x_in, void *x,
                             const void *w_scale = nullptr);

// act[i] = f16(f16(up_i) * silu(f16(gate_i))) with W rows interleaved (2i gate, 2i+1 up),
// after an RMSNorm prologue of x with norm_w.
int32_t launch_gate_up_swiglu(hipStream_t s, const void *x, const void *norm_w, float eps, const void *w,
                              int64_t ffn, int64_t dim, void *act, const void *w_scale = nullptr);

// lm_head with RMSNorm prologue and f16 logits, then the argmax of its per-workgroup partials
// (second launch), which writes the decode state.
struct LmHeadArgs {
    const void *x, *norm_w;
    float eps;
    const void *w;  // [vocab][dim]
    int64_t vocab, dim;
    void *logits;   // [vocab] f16
    void *partials; // [n_groups] (value, index)
    DecodeState *state;
    int64_t *ring;  // token ring (autoregressive loop), may be null
    const void *w_scale;  // Q8_0 lm_head scales (w is then int8), or null
    QFMat wq;             // Q4_0 / Q4_K / Q6_K lm_head (w and w_scale unused)
};
int32_t launch_lm_head_argmax(hipStream_t s, const LmHeadArgs &a);
int32_t launch_lm_head(hipStream_t s, const LmHeadArgs &a);
int32_t launch_argmax_finish(hipStream_t s, const void *partials, int64_t count, DecodeState *state, int64_t *ring,
                             int64_t *result);
int64_t lm_head_groups(int64_t vocab);

// ------------------------------------------------------------------ library GEMM (blas.hip)
// D[M][N] = A[M][K] W[N][K]^T on hipBLASLt: f16 operands, f32 accumulation, D in f16 or f32 (row
// major, leading dimension N); ws: workspace of ws_bytes. AESIR_ERR_UNSUPPORTED when the library
// has no algorithm for the shape (the caller then takes its own kernel).
int32_t blas_gemm_nt(aesir_ctx *ctx, hipStream_t s, const void *A, int64_t M, int64_t K, const void *W, int64_t N,
                     void *D, bool f32_out, void *ws, int64_t ws_bytes);

// ------------------------------------------------------------------ attention (attention.hip)
struct AttnArgs {
    const void *q;              // [nq * hd]
    const void *k, *v;          // row 0 of the key/value views
    int64_t k_stride, v_stride; // elements per row
    void *out;                  // [nq * hd]
    int64_t nq, nkv, hd;
    float scale;
    int64_t seq_len;            // >= 1, or 0 to read S = min(pos + 1, max_seq) from state
    const DecodeState *state;
    int64_t max_seq;
    float *part;                // partials [nq][max_split][hd + 2]
    int64_t max_split;          // <= 128
};
// Two launches: split-KV partials (register/LDS fast path for head_dim 64 and 128, generic
// LDS-tiled kernel otherwise), then the merge (one workgroup per query head).
int32_t launch_attention_decode(hipStream_t s, const AttnArgs &a);
int64_t attention_partial_floats(int64_t nq, int64_t hd, int64_t max_split);
// Split count for a KV view of up to max_positions rows.
int64_t attention_split_count(int64_t hd, int64_t max_positions);

// ------------------------------------------------------------------ elementwise (basic.hip)
int32_t launch_rmsnorm(hipStream_t s, void *T, int64_t rows, int64_t cols, const void *w, float eps);
int32_t launch_rope(hipStream_t s, void *Q, int64_t q_rows, int64_t q_cols, void *K, int64_t k_cols,
                    int64_t start_pos, int64_t head_dim, const void *table);
int32_t launch_silu(hipStream_t s, void *T, int64_t n);
int32_t launch_swiglu(hipStream_t s, void *up, void *gate, int64_t n);
int32_t launch_residual_add(hipStream_t s, void *x, const void *r, int64_t n);
int32_t launch_embed(hipStream_t s, const void *table, int64_t dim, int64_t token, const DecodeState *state,
                     void *x);
int32_t launch_kv_append(hipStream_t s, void *kc, void *vc, const void *k, const void *v, int64_t n);
int32_t launch_argmax(hipStream_t s, const void *logits, int64_t n, void *partials, int64_t max_parts,
                      int64_t *result);
int32_t launch_fill_normal(hipStream_t s, void *dst, int64_t n, int64_t cols, int64_t dst_stride, uint64_t seed,
                           uint64_t stream, float mean, float std);
// Q8_0 matrix init (quants [rows][cols] at q_stride bytes per row, f16 block scales at d_stride
// elements per row): q uniform in [-127, 127], d uniform in [0.5, 1.5) * std / 64.
int32_t launch_fill_q8_0(hipStream_t s, void *q, int64_t q_stride, void *d, int64_t d_stride, int64_t rows,
                         int64_t cols, uint64_t seed, uint64_t stream, float std);
int32_t launch_f32_to_f16(hipStream_t s, const float *src, void *dst, int64_t n);

// ------------------------------------------------------------------ Q8_0 (q8_0.hip)
int32_t launch_gemm_q8_0(hipStream_t s, const void *A, int64_t M, int64_t K, const void *blocks, int64_t N,
                         void *C);
int32_t launch_q8_0_matvec_f32(hipStream_t s, const void *blocks, int64_t N, int64_t K, const float *x,
                               float *y);

}  // namespace aesir
