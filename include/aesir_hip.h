/*
 * aesir_hip.h -- C ABI of libaesir_hip.so, the MI355X (gfx950) implementation of A.E.S.I.R.'s
 * Llama F16 forward path.
 *
 * Plain C: opaque handles, raw device pointers, int64 sizes, float scalars. No C++ or torch
 * types cross this boundary, so Mojo's external_call, ctypes, cgo or JNI can bind it directly.
 *
 * Every function returns int32_t: 0 (AESIR_OK) on success or a negative AESIR_ERR_* code, with
 * the message in aesir_last_error(). Where the reference raises, the message text is the
 * reference's own (paths below are relative to the reference repo's aesir_engine/ directory).
 * Where the reference returns silently on invalid input (flash_attention_gqa, silu), the call
 * returns AESIR_OK and leaves its output untouched.
 *
 * Ordering: all device work of one context runs in order on that context's single HIP stream.
 * Calls return after enqueueing, except those that hand a value back to the host
 * (aesir_argmax_f16, aesir_forward_pass, aesir_prefill, aesir_generate, aesir_memcpy_d2h,
 * aesir_ctx_synchronize), which wait for the stream. A context is not thread-safe, like the
 * reference engine (core/thread_pool.mojo:23-29 is a stub; nothing runs in parallel).
 */
#ifndef AESIR_HIP_H
#define AESIR_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AESIR_ABI_VERSION 1

#define AESIR_OK 0
#define AESIR_ERR_INVALID (-1)     /* invalid argument: non-positive dims, bad index, bad eps */
#define AESIR_ERR_SHAPE (-2)       /* shape mismatch between operands */
#define AESIR_ERR_EXHAUSTED (-3)   /* "MimirWell: memory pool exhausted" */
#define AESIR_ERR_HIP (-4)         /* HIP runtime failure (message names the call) */
#define AESIR_ERR_FORMAT (-5)      /* GGUF contract violation */
#define AESIR_ERR_IO (-6)          /* file open / mmap failure */
#define AESIR_ERR_UNSUPPORTED (-7) /* shape this build does not implement (message says which) */

/* GGML tensor type ids accepted by aesir_model_set_tensor (loader/gguf.mojo:17-19). */
#define AESIR_GGML_F32 0
#define AESIR_GGML_F16 1
/* GGML block_q8_0 {f16 d; int8 qs[32]} (34 bytes per 32 weights). The reference dequantizes it in
 * gemm_q8_0 (core/compute.mojo:1038-1065) but its loader rejects it (loader/gguf.mojo:450-463);
 * here it is also a model weight type (aesir_model_create_typed, aesir_model_load_gguf). */
#define AESIR_GGML_Q8_0 8
/* GGML block_q4_0 {f16 d; uint8 qs[16]} (18 bytes per 32 weights; byte i: element i in the low
 * nibble, element i + 16 in the high nibble). The reference's gemm_q4_0 / dequantize_q4_0
 * (core/compute.mojo:876-912, 266-280) fix the arithmetic: w = f16(f16(q - 8) * d). */
#define AESIR_GGML_Q4_0 2
/* GGML's K-quant super-blocks of 256 weights as GGUF files hold them (the ids the reference loader
 * names at loader/gguf.mojo:20-30): block_q4_K {f16 d; f16 dmin; uint8 scales[12]; uint8 qs[128]}
 * (144 bytes), w = d * sc * q - dmin * m with 6-bit sc, m per 32 weights; block_q6_K {uint8 ql[128];
 * uint8 qh[64]; int8 scales[16]; f16 d} (210 bytes), w = d * sc * (q - 32) with 6-bit q. The
 * reference's BlockQ4_K is a different, synthetic 32-weight block {f16 scale; f16 min_val;
 * uint8 qs[16]} (core/compute.mojo:84-98). Its BlockQ6_K has GGML's fields (:183-199), but its
 * decoder dequantize_q6_k_block (:508-527) ignores the scales and reads qh[(i + 128) / 2], past
 * qh's 64 entries, for every upper-half weight (:524); so the library follows GGML's layout and
 * formula for both. Weights are f16: a = f16(d * sc), b = f16(dmin * m), then Q4_K
 * w = f16(a * q - b) rounded once (GGML evaluates the formula in f32 and the reference has no
 * K-quant arithmetic for these blocks, so the library keeps the f16 value nearest the exact
 * a * q - b) and Q6_K w = f16(a * (q - 32)) (aesir_gemm_quant). */
#define AESIR_GGML_Q4_K 12
#define AESIR_GGML_Q6_K 14
/* The reference's other GGUF-block formats (loader/gguf.mojo:21-29): block_q4_1 {f16 d; f16 m;
 * uint8 qs[16]} (20 bytes / 32 weights), block_q5_0 {f16 d; uint8 qh[4]; uint8 qs[16]} (22),
 * block_q5_1 {f16 d; f16 m; uint8 qh[4]; uint8 qs[16]} (24), the reference's BlockQ4_1 / BlockQ5_0 /
 * BlockQ5_1 (core/compute.mojo:35-83), with its weights: Q4_1 w = f16(f16(q * d) + m), Q5_0
 * w = f16((q - 16) * d), Q5_1 w = f16(f16(q * d) + m) for the 4- or 5-bit q (compute.mojo:282-340,
 * each f16 operation rounded: these are the reference's own arithmetic on these very blocks, so
 * Q4_1 / Q5_1 keep its two roundings where the K-quants round once); and GGML's block_q2_K
 * (84 bytes / 256 weights), block_q3_K (110) and block_q5_K (176), whose f16 weights follow the
 * Q4_K / Q6_K rules: a = f16(d * sc), b = f16(dmin * m), w = f16(a * q - b) (Q2_K, Q5_K, one
 * rounding) or f16(a * q) (Q3_K, signed q). */
#define AESIR_GGML_Q4_1 3
#define AESIR_GGML_Q5_0 6
#define AESIR_GGML_Q5_1 7
#define AESIR_GGML_Q2_K 10
#define AESIR_GGML_Q3_K 11
#define AESIR_GGML_Q5_K 13

/* GPURealmType.AMD_ROCM_HIP (core/mimir_well.mojo:99): the realm id this library serves. */
#define AESIR_REALM_AMD_ROCM_HIP 1

typedef struct aesir_ctx aesir_ctx;
typedef struct aesir_kv aesir_kv;
typedef struct aesir_model aesir_model;

/* Thread-local message of the last failing call on this thread (empty string if none). */
const char *aesir_last_error(void);
int32_t aesir_abi_version(void);

/* ======================================================================= context + arena
 * One context = one GPU, one HIP stream and one hipMalloc'd HBM arena (the MimirWell).
 * Replaces MimirWell.__init__ (core/mimir_well.mojo:533-541), which allocates and zeroes a host
 * pool; here the pool is device memory, zeroed at creation. */
int32_t aesir_ctx_create(int32_t device, int64_t well_bytes, aesir_ctx **out);
/* Fails (AESIR_ERR_INVALID, context left intact) while a model created on it is alive: models hold
 * pointers into the context, so destroy them first. */
int32_t aesir_ctx_destroy(aesir_ctx *ctx);
int32_t aesir_ctx_synchronize(aesir_ctx *ctx);
/* The context's hipStream_t, for callers that interleave their own work. */
void *aesir_ctx_stream(aesir_ctx *ctx);
/* Device name (e.g. "gfx950"), compute-unit count and HBM bytes of the context's GPU. */
int32_t aesir_ctx_device_info(aesir_ctx *ctx, char *arch_out, int32_t arch_cap, int32_t *cu_count,
                              int64_t *hbm_bytes);

/* MimirWell.allocate (core/mimir_well.mojo:543-551): bump-allocates `elements` f16 elements
 * (2 bytes each, 256-byte aligned) and returns a device pointer. Raises
 * "MimirWell: allocation count must be positive" / "MimirWell: memory pool exhausted". */
int32_t aesir_well_allocate(aesir_ctx *ctx, int64_t elements, void **dev_ptr);
/* MimirWell.reset_kv_cache (core/mimir_well.mojo:562-566): "MimirWell: invalid reset offset". */
int32_t aesir_well_reset(aesir_ctx *ctx, int64_t offset);
/* MimirWell.offset / .capacity, in f16 elements (core/mimir_well.mojo:529-531). */
int64_t aesir_well_offset(const aesir_ctx *ctx);
int64_t aesir_well_capacity(const aesir_ctx *ctx);

/* Host<->device copies on the context stream (the reference's AMDGate.memcpy_* hooks,
 * core/amd_gate.mojo:71-111, which are no-ops there). d2h waits for completion. */
int32_t aesir_memcpy_h2d(aesir_ctx *ctx, void *dev_dst, const void *host_src, int64_t bytes);
int32_t aesir_memcpy_d2h(aesir_ctx *ctx, void *host_dst, const void *dev_src, int64_t bytes);
int32_t aesir_memcpy_d2d(aesir_ctx *ctx, void *dev_dst, const void *dev_src, int64_t bytes);

/* HIP-event timer on the context stream: start, then stop returns elapsed milliseconds. */
int32_t aesir_timer_start(aesir_ctx *ctx);
int32_t aesir_timer_stop(aesir_ctx *ctx, float *elapsed_ms);

/* ======================================================================= kernels
 * Tensors are RuneTensor views {device ptr, rows, cols}, row-major, f16 unless stated
 * (core/mimir_well.mojo:379-430). */

/* gemm_f16 (core/compute.mojo:1751-1854) and the AMD realm hook gemm_f16_gpu(...,
 * AMD_ROCM_HIP) -> AMDGate.launch_gemm_amd (core/compute.mojo:2554-2556,
 * core/amd_gate.mojo:113-167). C[m,n] = f16(sum_k f32(A[m,k]) * f32(B[n,k])), f32 accumulation.
 * One row of A runs the decode GEMV; two or more the matrix-core GEMM (a_cols a multiple of 64,
 * 16-byte aligned operands; other shapes the GEMV per row). Raises "gemm_f16: matrix dimensions
 * must be positive", "gemm_f16: inner matrix dimension
 * mismatch", "gemm_f16: output matrix shape mismatch". */
int32_t aesir_gemm_f16(aesir_ctx *ctx, const void *A, int64_t a_rows, int64_t a_cols, const void *B,
                       int64_t b_rows, int64_t b_cols, void *C, int64_t c_rows, int64_t c_cols);

/* rmsnorm (core/compute.mojo:2166-2204), in place on T [rows x cols]; weight has weight_size
 * elements. Raises "rmsnorm: tensor dimensions must be positive", "rmsnorm: weight dimension
 * mismatch", "rmsnorm: epsilon must be positive". */
int32_t aesir_rmsnorm_f16(aesir_ctx *ctx, void *T, int64_t rows, int64_t cols, const void *weight,
                          int64_t weight_size, float epsilon);

/* apply_rope (core/compute.mojo:2207-2244), in place on Q and K, adjacent-pair rotation,
 * row r at position start_pos + r. Raises the reference's four messages, plus
 * "apply_rope: K rows must cover Q rows" where the reference would index K out of bounds. */
int32_t aesir_rope_f16(aesir_ctx *ctx, void *Q, int64_t q_rows, int64_t q_cols, void *K, int64_t k_rows,
                       int64_t k_cols, int64_t start_pos, int64_t head_dim, float theta);

/* flash_attention_gqa (core/compute.mojo:1950-2015): one query row, keys/values views of
 * seq_len rows with row strides keys_cols/values_cols. Invalid inputs (seq_len <= 0, rows != 1,
 * counts <= 0, nq % nkv != 0) return AESIR_OK with output untouched, as the reference does.
 * head_dim above 256 returns AESIR_ERR_UNSUPPORTED. Split-KV with an fp32 online softmax. */
int32_t aesir_attn_gqa_decode(aesir_ctx *ctx, const void *query, int64_t query_rows, const void *keys,
                              int64_t keys_cols, const void *values, int64_t values_cols, void *output,
                              int64_t output_rows, int64_t seq_len, int64_t head_dim, int64_t nq,
                              int64_t nkv);

/* Allocation-free variant of aesir_attn_gqa_decode; it has no counterpart in the reference. It is
 * for callers that cannot allocate device memory: code under HIP graph capture, tight serving
 * loops and harnesses that forbid hipMalloc. It takes no context: work is enqueued on `stream`
 * (a hipStream_t; NULL is the null stream) of the calling thread's current device. Same
 * arguments, checks and results as aesir_attn_gqa_decode, with the split partials held in a
 * static 4 MiB device array per GPU (2^20 floats: nq * splits * (head_dim + 2) must fit; the
 * split count is halved until it does, and sizes that do not fit with one split are rejected
 * with AESIR_ERR_UNSUPPORTED). It calls no allocator. All calls on one GPU share that array:
 * calls that overlap on one GPU (two streams, or two host threads) race and must be ordered by
 * the caller. The first call on each device resolves the array's device address
 * (hipGetSymbolAddress) and must be made outside any stream capture; later calls may be captured
 * into a HIP graph, whose replays recompute every partial they read. */
int32_t aesir_attn_gqa_decode_static(void *stream, const void *query, int64_t query_rows, const void *keys,
                                     int64_t keys_cols, const void *values, int64_t values_cols, void *output,
                                     int64_t output_rows, int64_t seq_len, int64_t head_dim, int64_t nq,
                                     int64_t nkv);

/* silu (core/compute.mojo:2113-2126), in place; size <= 0 is a no-op. */
int32_t aesir_silu_f16(aesir_ctx *ctx, void *T, int64_t size);
/* SwiGLU as TransformerBlock.forward does it (core/inference.mojo:258-260): silu(gate) in
 * place, then up[i] = f16(up[i] * gate[i]). */
int32_t aesir_swiglu_f16(aesir_ctx *ctx, void *up, void *gate, int64_t size);
/* Residual add (core/inference.mojo:231-232, 272-273): x[i] = f16(x[i] + residual[i]). */
int32_t aesir_residual_add_f16(aesir_ctx *ctx, void *x, const void *residual, int64_t size);
/* Embedding row copy (core/inference.mojo:452-467): x = table[token]. Raises "Prompt token ID is
 * outside the embedding vocabulary". */
int32_t aesir_embed_f16(aesir_ctx *ctx, const void *table, int64_t vocab, int64_t dim, int64_t token,
                        void *x);
/* Greedy argmax (core/inference.mojo:508-515): floor f16(-10000), strict '>', lowest index
 * wins ties, NaN never chosen, 0 if nothing exceeds the floor. Waits; result in *index. */
int32_t aesir_argmax_f16(aesir_ctx *ctx, const void *logits, int64_t n, int64_t *index);

/* gemm_q8_0 (core/compute.mojo:1038-1065) reached through gemm_f16's quant dispatch (:1776-1778):
 * B is b_rows x a_cols weights as GGUF block_q8_0 {f16 d; int8 qs[32]} (34 bytes, packed).
 * w = f16(f16(q) * d); C = f16(sum f32(A) * f32(w)). a_cols must be a multiple of 32. */
int32_t aesir_gemm_q8_0(aesir_ctx *ctx, const void *A, int64_t a_rows, int64_t a_cols, const void *blocks,
                        int64_t b_rows, void *C, int64_t c_rows, int64_t c_cols);
/* The reference's quantized branch of gemm_f16 (core/compute.mojo:1763-1800) over packed GGUF
 * blocks of ggml_type: B is b_rows x a_cols weights, C[m, n] = f16(sum_k A[m, k] w[n, k]).
 * AESIR_GGML_Q4_0 / _Q4_1 / _Q5_0 / _Q5_1 follow gemm_q4_0 / _q4_1 / _q5_0 / _q5_1 (:876-1036;
 * w = f16(f16(q - 8) * d), f16(f16(q * d) + m), f16((q - 16) * d), f16(f16(q * d) + m));
 * AESIR_GGML_Q8_0 is aesir_gemm_q8_0; AESIR_GGML_Q4_K / _Q5_K / _Q6_K / _Q2_K / _Q3_K read GGML's
 * super-blocks with f16 weights in the f16 arithmetic of the reference's dequantize_q4_k_m /
 * dequantize_q6_k_block (:245-262, :508-527): w = f16(f16(d * sc) * q - f16(dmin * m)) (one fused
 * rounding; Q4_K, Q5_K, Q2_K) and w = f16(f16(d * sc) * q) (Q6_K with q - 32, Q3_K with its signed
 * q) (the reference's K-quant gemms read synthetic block layouts that no GGUF file holds). Raises
 * "gemm_q4_0: matrix dimensions must be positive", "...: inner dimension must be a multiple of
 * 32" (256 for the K-quants), "...: output matrix shape mismatch". Takes free well space for the
 * duration of the call: with a_rows < 16 and a_cols a multiple of 128 (at most 28672), or with
 * a_rows > 64 and a_cols a multiple of 128, the blocks are repacked into the library's tiled
 * planes (about the size of the blocks) for the decode GEMV per row or the matrix-core GEMM that
 * dequantizes in registers; otherwise an f16 copy of the weights (2 bytes per weight) for the F16
 * GEMM. */
int32_t aesir_gemm_quant(aesir_ctx *ctx, const void *A, int64_t a_rows, int64_t a_cols, const void *blocks,
                         int32_t ggml_type, int64_t b_rows, void *C, int64_t c_rows, int64_t c_cols);
/* Q8_0 block matvec with f32 activations and f32 output: y[n] = sum_k x[k] * d*q. Rows of
 * 64-512 blocks use exact integer dot products on x held as 30-bit fixed point per block: each
 * block's value is within 2^-30 * max|x_blk| * sum|d*q| of the exact block dot product (plus one
 * f32 rounding), and the block values are summed in f32. Other shapes use the f32 formula. An inf
 * or NaN in x propagates as in the f32 formula. */
int32_t aesir_q8_0_matvec_f32(aesir_ctx *ctx, const void *blocks, int64_t n_rows, int64_t k, const float *x,
                              float *y);

/* ======================================================================= sampler
 * sample_token_from_logits (core/sampler.mojo:217-305): the whole sampler stack on the device.
 * Parameter meaning as in the reference: temperature <= 0 or top_k == 1 is the greedy branch
 * (first maximum of the sanitized logits, suppressed ids at -1e9); otherwise the suppress mask,
 * repetition penalty (1 = off), frequency / presence penalties (0 = off) and temperature scale
 * every candidate, then top_k (> 0), top_p (< 1) and min_p (in (0, 1)) truncate the stably
 * sorted list, and RuneRNG.next_float32 drives the draw. */
typedef struct {
    float temperature;
    int64_t top_k;
    float top_p;
    float min_p;
    float repetition_penalty;
    float frequency_penalty;
    float presence_penalty;
} aesir_sampler_config;

/* logits: f16 [vocab] on the device; context / suppress: host token id lists; *rng_state: the
 * RuneRNG state (sampler.mojo:17-43), advanced only when the draw consumes a random number, as
 * the reference does. Waits; *token receives the sampled id (0 for vocab <= 0, as :232-233). */
int32_t aesir_sample_token(aesir_ctx *ctx, const void *logits, int64_t vocab, const aesir_sampler_config *cfg,
                           const int64_t *context, int64_t n_context, const int64_t *suppress, int64_t n_suppress,
                           uint64_t *rng_state, int64_t *token);
/* RuneRNG.next_u64 (core/sampler.mojo:34-37) on a host state: the mixer advances the state itself.
 * RuneRNG(seed) starts from seed, or from 0x9E3779B97F4A7C15 when seed is 0 (:25-29). */
uint64_t aesir_rune_rng_next(uint64_t *state);

/* ======================================================================= KV cache
 * KVCache (core/mimir_well.mojo:434-521): K and V each [num_layers][max_seq_len][hidden_dim]
 * f16, carved from the context's well. */
int32_t aesir_kv_create(aesir_ctx *ctx, int64_t max_seq_len, int64_t hidden_dim, int64_t num_layers,
                        aesir_kv **out);
int32_t aesir_kv_destroy(aesir_kv *kv); /* frees the descriptor; the memory belongs to the well */
/* KVCache.append (:488-501): writes key/val rows at slot pos % max_seq_len. */
int32_t aesir_kv_append(aesir_ctx *ctx, aesir_kv *kv, int64_t layer_idx, int64_t pos, const void *key,
                        int64_t key_size, const void *val, int64_t val_size);
/* KVCache.get_k_slice / get_v_slice (:503-521): device pointer of row 0 of the layer. */
int32_t aesir_kv_k_slice(const aesir_kv *kv, int64_t layer_idx, int64_t seq_len, void **dev_ptr);
int32_t aesir_kv_v_slice(const aesir_kv *kv, int64_t layer_idx, int64_t seq_len, void **dev_ptr);

/* ======================================================================= model + engine */
typedef struct {
    int64_t dim;        /* llama.embedding_length */
    int64_t n_layers;   /* llama.block_count */
    int64_t n_heads;    /* llama.attention.head_count */
    int64_t n_kv_heads; /* llama.attention.head_count_kv */
    int64_t ffn;        /* llama.feed_forward_length */
    int64_t vocab;      /* rows of token_embd.weight */
    int64_t ctx_len;    /* llama.context_length: KV cache rows */
    float rms_eps;      /* llama.attention.layer_norm_rms_epsilon (default 1e-5) */
    float rope_theta;   /* the reference always applies 10000 (core/inference.mojo:200) */
    int64_t bos_token_id;
    int64_t eos_token_id;
} aesir_model_config;

/* Lays out one model in the well: f16 weights (Q/K/V rows concatenated, gate/up rows
 * interleaved), norms, KV cache [layers][ctx_len][kv_dim] x2, decode workspace and the batched
 * prefill's workspace for chunks of R = min(ctx_len, 2048) rows: 2 x R x (5 dim + 2 kv_dim + ffn)
 * bytes of activations (151 MB for the Llama-3-8B shape) plus the K-split partials, plus
 * 4 x R x ffn bytes of gate/up products only when dim or ffn is not a multiple of 64 (the shapes
 * whose prefill GEMMs fall back to the GEMV path). A quantized model of a repacked type also holds
 * an f16 copy of its largest layer matrix for short prefill chunks (2 x 2 ffn x dim bytes). The
 * weights start zeroed. Validates the GGUFModelConfig contract (loader/gguf.mojo:133-149). */
int32_t aesir_model_create(aesir_ctx *ctx, const aesir_model_config *cfg, aesir_model **out);
/* aesir_model_create with a weight type for the seven matrix kinds (token_embd, output, attn_q/k/v,
 * attn_output, ffn_gate/up/down): AESIR_GGML_F16 (what aesir_model_create makes), AESIR_GGML_Q8_0,
 * or one of the GGML block types AESIR_GGML_Q4_0, _Q4_1, _Q5_0, _Q5_1, _Q2_K, _Q3_K, _Q4_K, _Q5_K,
 * _Q6_K. A Q8_0 model keeps each matrix as int8
 * quants [rows][cols] plus f16 block scales [rows][cols/32] in HBM (same fused row order as F16);
 * dim and ffn must be multiples of 32 (and at most 28672). Every weight is used as
 * w = f16(f16(q) * d), gemm_q8_0's rule (core/compute.mojo:1062-1063), so a Q8_0 model computes
 * what the F16 model holding the dequantized weights computes. A model of any other block type
 * keeps each matrix repacked into 16-weight records in 16-row x 128-weight tiles (nibble plane,
 * per-block scale planes, a fifth-bit or high-bit plane; Q2_K / Q3_K at GGUF's bit width: a 2-bit
 * crumb plane, plus Q3_K's third-bit plane); dim
 * and ffn must be multiples of 128 (32-weight blocks) or 256 (K-quants), at most 28672. Every type's
 * weights are the f16 values of aesir_gemm_quant's rules, so a model of any type computes what
 * the F16 model holding its read-back weights computes. Norm vectors stay f16. No reference
 * counterpart as a model (the reference loader has no quantized model path,
 * loader/gguf.mojo:450-463). */
int32_t aesir_model_create_typed(aesir_ctx *ctx, const aesir_model_config *cfg, int32_t weight_type,
                                 aesir_model **out);
/* aesir_model_create_typed with one type per matrix: tensor_types holds n_types = 2 + 7 * n_layers
 * ids in the order token_embd, output, then per layer attn_q, attn_k, attn_v, attn_output,
 * ffn_gate, ffn_up, ffn_down (each F16 or a type aesir_model_create_typed takes, with that
 * type's dim / ffn constraints). Each matrix keeps its own type in HBM, except the two fused
 * ones: a layer's Q/K/V (and its gate/up) matrix is stored in f16 when its parts differ in type,
 * each part dequantized at upload by its type's rule. aesir_model_set_tensor then takes each
 * tensor in its own type. This is the layout of GGUF files that mix types (Q4_K_M and the like). No reference
 * counterpart (the reference loader takes F16 files only, loader/gguf.mojo:450-463). */
int32_t aesir_model_create_mixed(aesir_ctx *ctx, const aesir_model_config *cfg, const int32_t *tensor_types,
                                 int64_t n_types, aesir_model **out);
/* aesir_model_weight_type's value for a model whose matrices differ in type. */
#define AESIR_WEIGHT_MIXED (-2)
/* Weight type of the model's matrices (AESIR_GGML_F16 or a GGML block type), or
 * AESIR_WEIGHT_MIXED when they differ (aesir_model_tensor_type gives each). */
int32_t aesir_model_weight_type(const aesir_model *model);
/* GGML type that aesir_model_set_tensor takes for the named tensor (norms: AESIR_GGML_F16, which
 * also takes F32); a negative error code for an unknown name. */
int32_t aesir_model_tensor_type(aesir_model *model, const char *name);
int32_t aesir_model_destroy(aesir_model *model);
int32_t aesir_model_get_config(const aesir_model *model, aesir_model_config *cfg);
/* Uploads one tensor by its GGUF name ("token_embd.weight", "blk.N.attn_q.weight", ...),
 * host data in GGUF order (rows x cols, cols fastest). F32 tensors are rounded to f16 as
 * loader/gguf.mojo:486-493 does. Shape and type are checked against
 * _validate_required_tensors (loader/gguf.mojo:567-628) with its messages. The matrices of a
 * quantized model take data of their type (aesir_model_tensor_type) as GGUF packs it: rows x
 * (cols/32) blocks of 34 (Q8_0), 18 (Q4_0), 20 (Q4_1), 22 (Q5_0) or 24 (Q5_1) bytes, rows x
 * (cols/256) blocks of 84 (Q2_K), 110 (Q3_K), 144 (Q4_K), 176 (Q5_K) or 210 (Q6_K) bytes. */
int32_t aesir_model_set_tensor(aesir_model *model, const char *name, const void *host_data, int64_t rows,
                               int64_t cols, int32_t ggml_type);
/* Reads a tensor back in GGUF order as f16 (for verification); quantized matrices come back
 * dequantized to the f16 weights the model multiplies: f16(q * d) (Q8_0), the rules of
 * aesir_gemm_quant for the other block types. */
int32_t aesir_model_get_tensor(aesir_model *model, const char *name, void *host_out, int64_t elements);
/* Device-side seeded random init: every weight N(0, std), every norm N(norm_mean, norm_std),
 * rounded to f16; element i of tensor t uses the same counter-based Box-Muller stream as the
 * test oracle's generator. For models too large to build on the host. Q8_0 matrices get
 * quants uniform in [-127, 127] and block scales uniform in [0.5, 1.5) * std / 64 (weights of
 * standard deviation near std); repacked matrices get uniform nibbles (and fifth or high bits)
 * with scales chosen for a standard deviation near std. */
int32_t aesir_model_init_random(aesir_model *model, uint64_t seed, float std, float norm_mean, float norm_std);
/* GGUFSeer.mmap_and_load (loader/gguf.mojo:664-690) + AesirEngine.__init__'s layer setup
 * (aesir.mojo:237-296): parses a GGUF v3 Llama F16 file, enforces the reference loader
 * contract, creates the model (KV rows = ctx_len_override if > 0, else llama.context_length)
 * and uploads every tensor into HBM. Beyond the reference loader each matrix may also be Q8_0,
 * Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q4_K, Q5_K or Q6_K, matrix by matrix (norms F32): a file
 * whose matrices share one type gives a model of that weight type (aesir_model_create_typed), a
 * file that mixes them (Q4_K_M and the like) the model aesir_model_create_mixed makes for its
 * types. Other matrix types are refused with "GGUF required tensor has an invalid type". */
int32_t aesir_model_load_gguf(aesir_ctx *ctx, const char *path, int64_t ctx_len_override, aesir_model **out);

/* GGUFSeer.inspect_metadata (loader/gguf.mojo:649-662), extended to the tensor table: parses and
 * validates a GGUF v3 file against the same contract as aesir_model_load_gguf (header, metadata,
 * tokenizer arrays, required tensors with shapes and types) without touching a GPU, and fills
 * *cfg (ctx_len = llama.context_length, rope_theta = 10000 as the reference applies).
 * *rope_freq_base receives llama.rope.freq_base when present (else 10000). */
int32_t aesir_gguf_inspect(const char *path, aesir_model_config *cfg, float *rope_freq_base);

/* forward_pass (core/inference.mojo:424-518): evaluates tokens[min(max(0,start_pos),n-1)] at
 * position start_pos through all layers (appending K/V at start_pos), then output norm, lm_head
 * and argmax. Waits; *next_token is the greedy token. */
int32_t aesir_forward_pass(aesir_model *model, const int64_t *tokens, int64_t n_tokens, int64_t start_pos,
                           int64_t *next_token);
/* The forward_pass overload without an explicit KVCache (core/inference.mojo:521-547): a fresh
 * cache of llama.context_length rows, then tokens[n_tokens - 1] evaluated at position
 * start_pos = n_tokens - 1 (0 for an empty list, which returns token 0). The reference carves the
 * new cache from never-used, zeroed well memory; here the model's own cache serves as that fresh
 * cache: rows [0, min(start_pos, ctx_len)) of every layer are cleared first (earlier contents
 * are lost). Waits; *next_token is the greedy token. */
int32_t aesir_forward_pass_no_cache(aesir_model *model, const int64_t *tokens, int64_t n_tokens,
                                    int64_t *next_token);
/* Batched prefill: the same result as forward_pass at each position start_pos .. start_pos +
 * n_tokens - 1 in turn (the per-position prefill loop of _run_generation, aesir.mojo:358-374),
 * computed with all positions of a chunk of up to 2048 rows going through each layer together: MFMA f16
 * GEMMs (f32 accumulate), causal GQA attention over the cache, K/V appended for every position.
 * tokens[i] is evaluated at position start_pos + i. Waits; *next_token is the greedy token after
 * the last position and aesir_model_logits returns its logits. f32 summation order differs from
 * the per-position path (results within the forward-pass tolerance). */
int32_t aesir_prefill(aesir_model *model, const int64_t *tokens, int64_t n_tokens, int64_t start_pos,
                      int64_t *next_token);
/* f16 logits [vocab] of the last forward pass, copied to the host. */
int32_t aesir_model_logits(aesir_model *model, void *host_out);

/* Device-autoregressive decode: starting from token at start_pos, runs n_steps forward passes
 * back to back, each consuming the previous step's argmax on the device (one HIP graph per
 * step when use_graph != 0). Tokens produced are copied to out_tokens[n_steps]; *elapsed_ms is
 * the HIP-event time of the n_steps passes on the context stream. */
int32_t aesir_decode_loop(aesir_model *model, int64_t token, int64_t start_pos, int64_t n_steps,
                          int32_t use_graph, int64_t *out_tokens, float *elapsed_ms);

/* Fills the first n_pos positions of every layer's K and V cache with N(0, std) f16 values from
 * the counter-based generator (seeded). No reference counterpart: it lets a throughput run start
 * at a given KV length without prefilling that many tokens. */
int32_t aesir_model_fill_kv_random(aesir_model *model, int64_t n_pos, uint64_t seed, float std);

/* Average per-launch device time (ms, HIP events on the context stream) of each decode-step
 * kernel, over `iters` rounds of back-to-back launches at position pos (the per-layer kernels
 * cycle through all layers). Order of times[]: 0 QKV+RoPE+KV append (layer 0 also embeds),
 * 1 attention (split-KV partials + merge), 2 O projection + residual, 3 RMSNorm + gate/up +
 * SwiGLU, 4 down projection + residual, 5 RMSNorm + lm_head, 6 argmax finish. n_times >= 7.
 * Leaves the decode workspace and the KV row at pos overwritten. */
int32_t aesir_model_kernel_times(aesir_model *model, int64_t pos, int32_t iters, float *times, int32_t n_times);

/* GenerationConfig subset that the token path needs (aesir.mojo:58-152). */
typedef struct {
    int64_t max_new_tokens;
    const int64_t *stop_tokens;
    int64_t n_stop_tokens;
    int32_t batched_prefill; /* 0: prefill by position as the reference does (aesir.mojo:358-374) */
} aesir_generation_config;

/* Stop reasons of generation_stop_reason (aesir.mojo:195-212). */
#define AESIR_STOP_EOS 0
#define AESIR_STOP_TOKEN 1
#define AESIR_STOP_LENGTH 2
#define AESIR_STOP_CONTEXT_EXHAUSTED 3

/* generation_stop_reason (aesir.mojo:195-212); returns -1 to continue. */
int32_t aesir_generation_stop_reason(int64_t token, int64_t eos_token_id, int64_t generated_count,
                                     int64_t max_new_tokens, const int64_t *stop_tokens, int64_t n_stop,
                                     int64_t next_position, int64_t context_length);
/* AesirEngine._run_generation (aesir.mojo:323-462) on token IDs: prefill, greedy decode loop,
 * stop policy. out_tokens must hold max_new_tokens entries. */
int32_t aesir_generate(aesir_model *model, const int64_t *prompt, int64_t n_prompt,
                       const aesir_generation_config *cfg, int64_t *out_tokens, int64_t *n_out,
                       int32_t *stop_reason);

#ifdef __cplusplus
}
#endif
#endif
