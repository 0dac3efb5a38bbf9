/*
 * aesir_oracle.h -- CPU restatement of A.E.S.I.R.'s verified Llama F16 forward path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP product path is
 * compared against. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * load it; the product library (libaesir_hip.so) never links, loads or calls it.
 *
 * Every function restates one reference function (paths relative to the reference repo
 * root, aesir_engine/ omitted where unambiguous) and keeps the reference's f16 rounding
 * points: f16 storage of every op output, f16 arithmetic for the RMSNorm scale, RoPE,
 * SiLU, SwiGLU and residual add, f32 accumulation where the reference accumulates in f32.
 * f16 values are carried as uint16_t bit patterns (IEEE binary16).
 *
 * Error returns follow the reference's raising functions: 0 on success, a negative code
 * on error, with the reference's message text available from ao_last_error().
 */
#ifndef AESIR_ORACLE_H
#define AESIR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    AO_OK = 0,
    AO_ERR_INVALID = -1,
    AO_ERR_SHAPE = -2,
    AO_ERR_EXHAUSTED = -3,
};

const char *ao_last_error(void);

/* ---- binary16 conversions (round to nearest even) ---- */
uint16_t ao_f32_to_f16(float f);
float ao_f16_to_f32(uint16_t h);
void ao_f32_to_f16_array(const float *src, uint16_t *dst, int64_t n);
void ao_f16_to_f32_array(const uint16_t *src, float *dst, int64_t n);
/* 1 when the AVX2/F16C build of the 16-lane loops is in use (same arithmetic either way). */
int ao_simd_enabled(void);

/* ---- kernels (compute.mojo / inference.mojo) ---- */
int ao_gemm_f16(const uint16_t *A, int64_t a_rows, int64_t a_cols, const uint16_t *B, int64_t b_rows,
                int64_t b_cols, uint16_t *C, int64_t c_rows, int64_t c_cols);
int ao_rmsnorm_f16(uint16_t *T, int64_t rows, int64_t cols, const uint16_t *w, int64_t w_size, float eps);
int ao_rope_f16(uint16_t *Q, int64_t q_rows, int64_t q_cols, uint16_t *K, int64_t k_rows, int64_t k_cols,
                int64_t start_pos, int64_t head_dim, float theta);
void ao_attn_gqa(const uint16_t *q, int64_t q_rows, const uint16_t *keys, int64_t keys_cols,
                 const uint16_t *values, int64_t values_cols, uint16_t *out, int64_t out_rows,
                 int64_t seq_len, int64_t head_dim, int64_t nq, int64_t nkv);
void ao_silu_f16(uint16_t *T, int64_t size);
void ao_mul_f16(uint16_t *up, const uint16_t *gate, int64_t size);
void ao_residual_add_f16(uint16_t *x, const uint16_t *residual, int64_t size);
int64_t ao_argmax_f16(const uint16_t *logits, int64_t n);
int64_t ao_greedy_sample_f16(const uint16_t *logits, int64_t n, const int64_t *suppress, int64_t n_suppress);
/* sample_token_from_logits (sampler.mojo:217-305). ao_sampler_config holds its parameters. */
typedef struct {
    float temperature;
    int64_t top_k;
    float top_p;
    float min_p;
    float repetition_penalty;
    float frequency_penalty;
    float presence_penalty;
} ao_sampler_config;
/* The candidate list after the mask, penalties, temperature and truncations (ids and f32
 * logits in candidate order); returns its length. */
int64_t ao_sample_candidates_f16(const uint16_t *logits, int64_t vocab, const ao_sampler_config *cfg,
                                 const int64_t *context, int64_t n_context, const int64_t *suppress,
                                 int64_t n_suppress, int64_t *ids_out, float *logits_out);
/* The sampled token; advances *rng_state when the draw consumes a random number. */
int64_t ao_sample_token_f16(const uint16_t *logits, int64_t vocab, const ao_sampler_config *cfg,
                            const int64_t *context, int64_t n_context, const int64_t *suppress,
                            int64_t n_suppress, uint64_t *rng_state);
float ao_rune_rng_next_float32(uint64_t *state);
int ao_gemm_q8_0(const uint16_t *A, int64_t a_rows, int64_t a_cols, const uint8_t *blocks, int64_t b_rows,
                 uint16_t *C, int64_t c_rows, int64_t c_cols);
void ao_dequantize_q8_0(const uint8_t *blocks, uint16_t *out, int64_t n_blocks);
/* gemm_q4_0 / dequantize_q4_0 (compute.mojo:876-912, 266-280) on GGUF block_q4_0 (18 bytes). */
int ao_gemm_q4_0(const uint16_t *A, int64_t a_rows, int64_t a_cols, const uint8_t *blocks, int64_t b_rows,
                 uint16_t *C, int64_t c_rows, int64_t c_cols);
void ao_dequantize_q4_0(const uint8_t *blocks, uint16_t *out, int64_t n_blocks);
/* GGML block_q4_K (144 bytes) / block_q6_K (210 bytes) super-blocks of 256 weights, dequantized
 * to f32 (GGML's published format; see aesir_oracle.c). */
void ao_dequantize_q4_k(const uint8_t *blocks, float *out, int64_t n_blocks);
void ao_dequantize_q6_k(const uint8_t *blocks, float *out, int64_t n_blocks);
void ao_dequantize_q4_k_f16(const uint8_t *blocks, uint16_t *out, int64_t n_blocks);
void ao_dequantize_q6_k_f16(const uint8_t *blocks, uint16_t *out, int64_t n_blocks);
/* GGUF block_q4_1 / block_q5_0 / block_q5_1 (GGML types 3, 6, 7; 20, 22, 24 bytes per 32 weights):
 * dequantize_q4_1 / _q5_0 / _q5_1 and gemm_q4_1 / _q5_0 / _q5_1 (compute.mojo:282-340, 914-1036). */
int ao_dequantize_legacy(int type, const uint8_t *blocks, uint16_t *out, int64_t n_blocks);
int ao_gemm_legacy(int type, const uint16_t *A, int64_t a_rows, int64_t a_cols, const uint8_t *blocks, int64_t b_rows,
                   uint16_t *C, int64_t c_rows, int64_t c_cols);
/* GGML block_q2_K / block_q3_K / block_q5_K (types 10, 11, 13; 84, 110, 176 bytes per 256 weights)
 * to GGML's f32 weights, and to the library's f16 weights. */
int ao_dequantize_kquant(int type, const uint8_t *blocks, float *out, int64_t n_blocks);
int ao_dequantize_kquant_f16(int type, const uint8_t *blocks, uint16_t *out, int64_t n_blocks);

/* ---- KV cache (mimir_well.mojo:434-521) over caller-owned buffers ---- */
typedef struct {
    uint16_t *k; /* [num_layers * max_seq][kv_dim] */
    uint16_t *v;
    int64_t max_seq, kv_dim, num_layers;
} ao_kv;
int ao_kv_append(ao_kv *kv, int64_t layer, int64_t pos, const uint16_t *key, int64_t key_size,
                 const uint16_t *val, int64_t val_size);
int ao_kv_slice(const ao_kv *kv, int64_t layer, int64_t seq_len, const uint16_t **k_out,
                const uint16_t **v_out);

/* ---- model + forward pass (inference.mojo:143-275, 424-518) ---- */
typedef struct {
    int64_t dim, n_layers, n_heads, n_kv_heads, ffn, vocab, ctx_len;
    float eps;
    float theta;
} ao_config;

typedef struct {
    ao_config cfg;
    const uint16_t *token_embd;  /* [vocab][dim] */
    const uint16_t *output_norm; /* [dim] */
    const uint16_t *output;      /* [vocab][dim] */
    const uint16_t **attn_norm;  /* per layer [dim] */
    const uint16_t **wq, **wk, **wv, **wo;
    const uint16_t **ffn_norm;
    const uint16_t **w_gate, **w_up, **w_down;
} ao_model;

/* scratch must hold ao_forward_scratch_elems(cfg) f16 elements. logits_out (may be NULL)
 * receives the f16 logits of this position. */
int64_t ao_forward_scratch_elems(const ao_config *cfg);
int ao_forward_pass(const ao_model *m, ao_kv *kv, const int64_t *tokens, int64_t n_tokens, int64_t start_pos,
                    uint16_t *scratch, uint16_t *logits_out, int64_t *next_token);
/* Runs only the first n_layers_run blocks plus the head (used to time a bounded CPU sample). */
int ao_forward_partial(const ao_model *m, ao_kv *kv, const int64_t *tokens, int64_t n_tokens,
                       int64_t start_pos, int64_t n_layers_run, uint16_t *scratch, uint16_t *logits_out,
                       int64_t *next_token);

/* aesir.mojo:195-212 */
int ao_generation_stop_reason(int64_t token, int64_t eos, int64_t generated_count, int64_t max_new,
                              const int64_t *stop_tokens, int64_t n_stop, int64_t next_position,
                              int64_t ctx_len);
/* aesir.mojo:323-462 without the tokenizer: prompt token IDs in, generated IDs out.
 * stop reason codes: 0 eos, 1 stop_token, 2 length, 3 context_exhausted. */
int ao_generate(const ao_model *m, ao_kv *kv, const int64_t *prompt, int64_t n_prompt, int64_t max_new,
                int64_t eos, const int64_t *stop_tokens, int64_t n_stop, uint16_t *scratch, int64_t *out_tokens,
                int64_t *n_out, int32_t *stop_reason, uint16_t *last_logits);

/* ---- synthetic inputs ---- */
/* RuneRNG (sampler.mojo:17-43): SplitMix64-style mixer applied to its own state. */
uint64_t ao_rune_rng_next(uint64_t *state);
/* Counter-based N(mean, std) fill (Box-Muller over the RuneRNG mixer), rounded to f16. */
void ao_fill_normal_f16(uint16_t *dst, int64_t n, uint64_t seed, uint64_t stream, float mean, float std);
void ao_fill_normal_f32(float *dst, int64_t n, uint64_t seed, uint64_t stream, float mean, float std);

#ifdef __cplusplus
}
#endif
#endif
