// C-ABI entry points of the per-op kernel API (the gemm_f16 / rmsnorm / apply_rope /
// flash_attention_gqa / silu / KVCache surface of core/compute.mojo and core/mimir_well.mojo).
// Each validates exactly as the reference function does, with the reference's message text,
// then enqueues the gfx950 kernel on the context stream.
#include <cmath>
#include <mutex>

#include "common.hpp"
#include "kernels.hpp"

using namespace aesir;

extern "C" {

int32_t aesir_gemm_f16(aesir_ctx *ctx, const void *A, int64_t a_rows, int64_t a_cols, const void *B,
                       int64_t b_rows, int64_t b_cols, void *C, int64_t c_rows, int64_t c_cols) {
    AESIR_TRY(bind(ctx));
    // compute.mojo:1756-1761
    if (a_rows <= 0 || a_cols <= 0 || b_rows <= 0 || b_cols <= 0)
        return fail(AESIR_ERR_INVALID, "gemm_f16: matrix dimensions must be positive");
    if (a_cols != b_cols) return fail(AESIR_ERR_SHAPE, "gemm_f16: inner matrix dimension mismatch");
    if (c_rows != a_rows || c_cols != b_rows) return fail(AESIR_ERR_SHAPE, "gemm_f16: output matrix shape mismatch");
    if (!A || !B || !C) return fail(AESIR_ERR_INVALID, "gemm_f16: null tensor pointer");
    // One row of A: the decode GEMV. More rows: the matrix-core GEMM, which reads B once for all
    // rows (the GEMV would read it once per row); shapes it does not tile fall back to the GEMV.
    if (a_rows >= 2) return launch_gemm_f16_mfma(ctx, A, a_rows, a_cols, B, b_rows, C);
    return launch_gemm_f16(ctx, A, a_rows, a_cols, B, b_rows, C);
}

int32_t aesir_rmsnorm_f16(aesir_ctx *ctx, void *T, int64_t rows, int64_t cols, const void *weight,
                          int64_t weight_size, float epsilon) {
    AESIR_TRY(bind(ctx));
    // compute.mojo:2172-2177
    if (rows <= 0 || cols <= 0) return fail(AESIR_ERR_INVALID, "rmsnorm: tensor dimensions must be positive");
    if (weight_size < cols) return fail(AESIR_ERR_SHAPE, "rmsnorm: weight dimension mismatch");
    if (!(epsilon > 0.0f)) return fail(AESIR_ERR_INVALID, "rmsnorm: epsilon must be positive");
    if (!T || !weight) return fail(AESIR_ERR_INVALID, "rmsnorm: null tensor pointer");
    return launch_rmsnorm(ctx->stream, T, rows, cols, weight, epsilon);
}

int32_t aesir_rope_f16(aesir_ctx *ctx, void *Q, int64_t q_rows, int64_t q_cols, void *K, int64_t k_rows,
                       int64_t k_cols, int64_t start_pos, int64_t head_dim, float theta) {
    AESIR_TRY(bind(ctx));
    // compute.mojo:2212-2219
    if (start_pos < 0) return fail(AESIR_ERR_INVALID, "apply_rope: start_pos cannot be negative");
    if (head_dim <= 0 || head_dim % 2 != 0) return fail(AESIR_ERR_INVALID, "apply_rope: head_dim must be positive and even");
    if (q_cols % head_dim != 0 || k_cols % head_dim != 0)
        return fail(AESIR_ERR_SHAPE, "apply_rope: tensor columns must be a multiple of head_dim");
    if (q_rows <= 0 || k_rows <= 0) return fail(AESIR_ERR_INVALID, "apply_rope: tensor dimensions must be positive");
    if (k_rows < q_rows) return fail(AESIR_ERR_SHAPE, "apply_rope: K rows must cover Q rows");
    if (!Q || !K) return fail(AESIR_ERR_INVALID, "apply_rope: null tensor pointer");
    const void *table = nullptr;
    AESIR_TRY(rope_table(ctx, theta, head_dim, start_pos + q_rows, &table));
    return launch_rope(ctx->stream, Q, q_rows, q_cols, K, k_cols, start_pos, head_dim, table);
}

}  // extern "C"

// Validation and argument set-up shared by the two attention entry points. *skip is set for the
// inputs on which the reference returns silently (compute.mojo:1961-1966); the split count is
// halved until the partials fit `part_cap` floats.
static int32_t attn_args_for_call(const void *query, int64_t query_rows, const void *keys, int64_t keys_cols,
                                  const void *values, int64_t values_cols, void *output, int64_t output_rows,
                                  int64_t seq_len, int64_t head_dim, int64_t nq, int64_t nkv, int64_t part_cap,
                                  const char *scratch_name, AttnArgs *out, bool *skip) {
    *skip = true;
    if (seq_len <= 0 || query_rows != 1 || output_rows != 1) return AESIR_OK;
    if (nq <= 0 || nkv <= 0 || head_dim <= 0) return AESIR_OK;
    if (nq % nkv != 0) return AESIR_OK;
    *skip = false;
    if (!query || !keys || !values || !output) return fail(AESIR_ERR_INVALID, "flash_attention_gqa: null tensor pointer");
    if (nkv * head_dim > keys_cols || nkv * head_dim > values_cols)
        return fail(AESIR_ERR_SHAPE, "flash_attention_gqa: key/value rows narrower than kv_heads * head_dim");
    AttnArgs a{};
    a.q = query;
    a.k = keys;
    a.v = values;
    a.k_stride = keys_cols;
    a.v_stride = values_cols;
    a.out = output;
    a.nq = nq;
    a.nkv = nkv;
    a.hd = head_dim;
    a.scale = (float)(1.0 / std::pow((double)head_dim, 0.5));  // compute.mojo:1968
    a.seq_len = seq_len;
    a.state = nullptr;
    a.max_seq = seq_len;
    int64_t max_split = attention_split_count(head_dim, seq_len);
    while (max_split > 1 && attention_partial_floats(nq, head_dim, max_split) > part_cap) max_split >>= 1;
    if (attention_partial_floats(nq, head_dim, max_split) > part_cap)
        return fail(AESIR_ERR_UNSUPPORTED, "flash_attention_gqa: %lld heads x %lld dims exceed the %s of %lld floats",
                    (long long)nq, (long long)head_dim, scratch_name, (long long)part_cap);
    a.max_split = max_split;
    *out = a;
    return AESIR_OK;
}

// ------------------------------------------------------------------ allocation-free attention
//
// Scratch of aesir_attn_gqa_decode_static: the split partials (m, l, acc) live in this
// file-scope array, one copy per GPU for the life of the process, so that entry point calls no
// allocator. Host code never passes `scratch` itself (in host code it names a host-side stand-in):
// the device address of each GPU's copy comes from hipGetSymbolAddress, taken once per device on
// that device's first call, and only that address reaches kernels.
constexpr int64_t kStaticAttnFloats = (int64_t)1 << 20;  // 4 MiB per GPU
static __device__ __align__(256) float scratch[kStaticAttnFloats];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch_ptr[kMaxScratchDevices];  // device address of `scratch`, by device ordinal
}  // namespace

static int32_t static_attn_scratch(float **out) {
    int dev = 0;
    AESIR_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxScratchDevices)
        return fail(AESIR_ERR_UNSUPPORTED, "flash_attention_gqa (static): device ordinal %d exceeds %d", dev,
                    kMaxScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(AESIR_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = (float *)p;
    }
    *out = g_scratch_ptr[dev];
    return AESIR_OK;
}

extern "C" {

int32_t aesir_attn_gqa_decode(aesir_ctx *ctx, const void *query, int64_t query_rows, const void *keys,
                              int64_t keys_cols, const void *values, int64_t values_cols, void *output,
                              int64_t output_rows, int64_t seq_len, int64_t head_dim, int64_t nq, int64_t nkv) {
    AESIR_TRY(bind(ctx));
    AttnArgs a{};
    bool skip = true;
    AESIR_TRY(attn_args_for_call(query, query_rows, keys, keys_cols, values, values_cols, output, output_rows, seq_len,
                                 head_dim, nq, nkv, ctx->scratch.attn_part_floats, "context scratch", &a, &skip));
    if (skip) return AESIR_OK;
    a.part = ctx->scratch.attn_part;
    return launch_attention_decode(ctx->stream, a);
}

int32_t aesir_attn_gqa_decode_static(void *stream, const void *query, int64_t query_rows, const void *keys,
                                     int64_t keys_cols, const void *values, int64_t values_cols, void *output,
                                     int64_t output_rows, int64_t seq_len, int64_t head_dim, int64_t nq, int64_t nkv) {
    clear_error();
    AttnArgs a{};
    bool skip = true;
    AESIR_TRY(attn_args_for_call(query, query_rows, keys, keys_cols, values, values_cols, output, output_rows, seq_len,
                                 head_dim, nq, nkv, kStaticAttnFloats, "static scratch", &a, &skip));
    if (skip) return AESIR_OK;
    float *part = nullptr;
    AESIR_TRY(static_attn_scratch(&part));
    a.part = part;
    return launch_attention_decode((hipStream_t)stream, a);
}

int32_t aesir_silu_f16(aesir_ctx *ctx, void *T, int64_t size) {
    AESIR_TRY(bind(ctx));
    if (size <= 0) return AESIR_OK;  // compute.mojo:2116-2117
    if (!T) return fail(AESIR_ERR_INVALID, "silu: null tensor pointer");
    return launch_silu(ctx->stream, T, size);
}

int32_t aesir_swiglu_f16(aesir_ctx *ctx, void *up, void *gate, int64_t size) {
    AESIR_TRY(bind(ctx));
    if (size <= 0) return AESIR_OK;
    if (!up || !gate) return fail(AESIR_ERR_INVALID, "swiglu: null tensor pointer");
    return launch_swiglu(ctx->stream, up, gate, size);
}

int32_t aesir_residual_add_f16(aesir_ctx *ctx, void *x, const void *residual, int64_t size) {
    AESIR_TRY(bind(ctx));
    if (size <= 0) return AESIR_OK;
    if (!x || !residual) return fail(AESIR_ERR_INVALID, "residual_add: null tensor pointer");
    return launch_residual_add(ctx->stream, x, residual, size);
}

int32_t aesir_embed_f16(aesir_ctx *ctx, const void *table, int64_t vocab, int64_t dim, int64_t token, void *x) {
    AESIR_TRY(bind(ctx));
    if (!table || !x) return fail(AESIR_ERR_INVALID, "Inference requires token_embd.weight");
    if (token < 0 || token >= vocab) return fail(AESIR_ERR_INVALID, "Prompt token ID is outside the embedding vocabulary");
    if (dim <= 0) return fail(AESIR_ERR_INVALID, "embedding: dimension must be positive");
    return launch_embed(ctx->stream, table, dim, token, nullptr, x);
}

int32_t aesir_argmax_f16(aesir_ctx *ctx, const void *logits, int64_t n, int64_t *index) {
    AESIR_TRY(bind(ctx));
    if (!index) return fail(AESIR_ERR_INVALID, "argmax: null output");
    if (n <= 0) {  // the reference's loop does not run: best_token stays 0
        *index = 0;
        return AESIR_OK;
    }
    if (!logits) return fail(AESIR_ERR_INVALID, "argmax: null logits");
    if (n > 2147483647) return fail(AESIR_ERR_UNSUPPORTED, "argmax: more than 2^31-1 logits");
    AESIR_TRY(launch_argmax(ctx->stream, logits, n, ctx->scratch.argmax_part, ctx->scratch.argmax_part_entries,
                            ctx->scratch.result));
    AESIR_HIP_TRY(hipMemcpyAsync(ctx->pinned_i64, ctx->scratch.result, sizeof(int64_t), hipMemcpyDeviceToHost, ctx->stream));
    AESIR_HIP_TRY(hipStreamSynchronize(ctx->stream));
    *index = ctx->pinned_i64[0];
    return AESIR_OK;
}

int32_t aesir_gemm_q8_0(aesir_ctx *ctx, const void *A, int64_t a_rows, int64_t a_cols, const void *blocks,
                        int64_t b_rows, void *C, int64_t c_rows, int64_t c_cols) {
    AESIR_TRY(bind(ctx));
    // compute.mojo:1039-1044
    if (a_rows <= 0 || a_cols <= 0 || b_rows <= 0) return fail(AESIR_ERR_INVALID, "gemm_q8_0: matrix dimensions must be positive");
    if (a_cols % 32 != 0) return fail(AESIR_ERR_SHAPE, "gemm_q8_0: inner dimension must be a multiple of 32");
    if (c_rows != a_rows || c_cols != b_rows) return fail(AESIR_ERR_SHAPE, "gemm_q8_0: output matrix shape mismatch");
    if (!A || !blocks || !C) return fail(AESIR_ERR_INVALID, "gemm_q8_0: null tensor pointer");
    return launch_gemm_q8_0(ctx->stream, A, a_rows, a_cols, blocks, b_rows, C);
}

int32_t aesir_gemm_quant(aesir_ctx *ctx, const void *A, int64_t a_rows, int64_t a_cols, const void *blocks,
                         int32_t ggml_type, int64_t b_rows, void *C, int64_t c_rows, int64_t c_cols) {
    AESIR_TRY(bind(ctx));
    if (ggml_type == AESIR_GGML_Q8_0) return aesir_gemm_q8_0(ctx, A, a_rows, a_cols, blocks, b_rows, C, c_rows, c_cols);
    const int64_t blk = gguf_block_elems(ggml_type);
    if (blk == 0)
        return fail(AESIR_ERR_UNSUPPORTED,
                    "gemm_quant: GGML type %d is not Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K or Q6_K",
                    (int)ggml_type);
    const char *nm = "gemm_q6_k";
    switch (ggml_type) {
        case AESIR_GGML_Q4_0: nm = "gemm_q4_0"; break;
        case AESIR_GGML_Q4_1: nm = "gemm_q4_1"; break;
        case AESIR_GGML_Q5_0: nm = "gemm_q5_0"; break;
        case AESIR_GGML_Q5_1: nm = "gemm_q5_1"; break;
        case AESIR_GGML_Q2_K: nm = "gemm_q2_k"; break;
        case AESIR_GGML_Q3_K: nm = "gemm_q3_k"; break;
        case AESIR_GGML_Q4_K: nm = "gemm_q4_k"; break;
        case AESIR_GGML_Q5_K: nm = "gemm_q5_k"; break;
        default: break;
    }
    // compute.mojo:877-882 (gemm_q4_0's checks; gemm_q4_1 / _q5_0 / _q5_1 and the K-quant twins
    // raise the same)
    if (a_rows <= 0 || a_cols <= 0 || b_rows <= 0) return fail(AESIR_ERR_INVALID, "%s: matrix dimensions must be positive", nm);
    if (a_cols % blk != 0)
        return fail(AESIR_ERR_SHAPE, "%s: inner dimension must be a multiple of %lld", nm, (long long)blk);
    if (c_rows != a_rows || c_cols != b_rows) return fail(AESIR_ERR_SHAPE, "%s: output matrix shape mismatch", nm);
    if (!A || !blocks || !C) return fail(AESIR_ERR_INVALID, "%s: null tensor pointer", nm);
    // Fewer than 16 rows of A on whole 128-weight segments of a repacked type: the blocks are
    // repacked into the tiled planes and each row runs the decode GEMV; more than 64 rows on whole
    // 128-weight segments: the same planes on the wide-tile matrix-core GEMM, which dequantizes
    // them in registers. Otherwise the blocks are dequantized to f16 (the same values) for the F16
    // GEMM, on the matrix cores from 2 rows. Both take free well space for this call, released after enqueueing (later work on the
    // stream runs after these kernels).
    // Both repacked-plane routes read A with 16-byte loads (the GEMV stages x with them, the wide
    // kernel copies A into LDS with them): an A that is not 16-byte aligned (an offset view) takes
    // the dequantize-then-F16 route, which checks its own alignment.
    const int64_t K = a_cols, N = b_rows, mark = ctx->well_offset;
    int32_t rc = AESIR_OK;
    const bool a16 = ((uintptr_t)A & 15) == 0;
    const bool wide = a16 && qf_type(ggml_type) && K % 128 == 0 && gemm_qf_wide_ok(a_rows, K, N);
    if ((a16 && a_rows < 16 && qf_type(ggml_type) && qf_gemv_ok(K)) || wide) {
        QFMat w;
        w.type = ggml_type;
        void *planes[4] = {nullptr, nullptr, nullptr, nullptr};
        for (int plane = 0; plane < 4 && rc == AESIR_OK; plane++) {
            const int64_t rb = qf_plane_row_bytes(ggml_type, plane, K);
            if (rb > 0) rc = well_alloc_bytes(ctx, mul_checked(qf_rows_alloc(N), rb), &planes[plane]);
        }
        w.nib = planes[0];
        w.hb = planes[1];
        w.s0 = planes[2];
        w.s1 = planes[3];
        if (rc == AESIR_OK) rc = launch_qf_repack(ctx->stream, ggml_type, blocks, N, K, w, 1);
        if (wide && rc == AESIR_OK) rc = launch_gemm_qf_mfma(ctx, A, a_rows, K, w, N, C);
        for (int64_t r = 0; !wide && r < a_rows && rc == AESIR_OK; r++)
            rc = launch_qf_gemv_store(ctx->stream, w, N, K, (const uint16_t *)A + r * K, (uint16_t *)C + r * N);
    } else {
        void *wf = nullptr;
        rc = well_alloc_bytes(ctx, mul_checked(N, K, 2), &wf);
        if (rc == AESIR_OK) rc = launch_gguf_dequant(ctx->stream, ggml_type, blocks, N, K, wf, K);
        if (rc == AESIR_OK)
            rc = a_rows >= 2 ? launch_gemm_f16_mfma(ctx, A, a_rows, K, wf, N, C) : launch_gemm_f16(ctx, A, a_rows, K, wf, N, C);
    }
    ctx->well_offset = mark;
    return rc;
}

int32_t aesir_q8_0_matvec_f32(aesir_ctx *ctx, const void *blocks, int64_t n_rows, int64_t k, const float *x, float *y) {
    AESIR_TRY(bind(ctx));
    if (n_rows <= 0 || k <= 0) return fail(AESIR_ERR_INVALID, "q8_0_matvec: matrix dimensions must be positive");
    if (k % 32 != 0) return fail(AESIR_ERR_SHAPE, "q8_0_matvec: inner dimension must be a multiple of 32");
    if (!blocks || !x || !y) return fail(AESIR_ERR_INVALID, "q8_0_matvec: null tensor pointer");
    return launch_q8_0_matvec_f32(ctx->stream, blocks, n_rows, k, x, y);
}

// ------------------------------------------------------------------ KV cache

int32_t aesir_kv_create(aesir_ctx *ctx, int64_t max_seq_len, int64_t hidden_dim, int64_t num_layers, aesir_kv **out) {
    AESIR_TRY(bind(ctx));
    if (!out) return fail(AESIR_ERR_INVALID, "KVCache: null output handle");
    // mimir_well.mojo:455-456
    if (max_seq_len <= 0 || hidden_dim <= 0 || num_layers <= 0) return fail(AESIR_ERR_INVALID, "KVCache: dimensions must be positive");
    const int64_t total = num_layers * max_seq_len * hidden_dim;
    void *k = nullptr, *v = nullptr;
    AESIR_TRY(aesir_well_allocate(ctx, total, &k));
    AESIR_TRY(aesir_well_allocate(ctx, total, &v));
    auto *kv = new aesir_kv();
    kv->ctx = ctx;
    kv->k = (uint16_t *)k;
    kv->v = (uint16_t *)v;
    kv->max_seq = max_seq_len;
    kv->hidden_dim = hidden_dim;
    kv->num_layers = num_layers;
    *out = kv;
    return AESIR_OK;
}

int32_t aesir_kv_destroy(aesir_kv *kv) {
    delete kv;
    return AESIR_OK;
}

int32_t aesir_kv_append(aesir_ctx *ctx, aesir_kv *kv, int64_t layer_idx, int64_t pos, const void *key, int64_t key_size,
                        const void *val, int64_t val_size) {
    AESIR_TRY(bind(ctx));
    if (!kv) return fail(AESIR_ERR_INVALID, "KVCache.append: null cache");
    // mimir_well.mojo:490-495
    if (layer_idx < 0 || layer_idx >= kv->num_layers) return fail(AESIR_ERR_INVALID, "KVCache.append: layer_idx out of bounds");
    if (pos < 0) return fail(AESIR_ERR_INVALID, "KVCache.append: pos must be non-negative");
    if (key_size < kv->hidden_dim || val_size < kv->hidden_dim) return fail(AESIR_ERR_SHAPE, "KVCache.append: key/val width mismatch");
    const int64_t slot = pos % kv->max_seq;
    const int64_t off = (layer_idx * kv->max_seq + slot) * kv->hidden_dim;
    return launch_kv_append(ctx->stream, kv->k + off, kv->v + off, key, val, kv->hidden_dim);
}

static int32_t kv_slice(const aesir_kv *kv, int64_t layer_idx, int64_t seq_len, bool is_k, void **ptr) {
    const char *nm = is_k ? "get_k_slice" : "get_v_slice";
    if (!kv || !ptr) return fail(AESIR_ERR_INVALID, "KVCache.%s: null argument", nm);
    // mimir_well.mojo:506-509, 515-518
    if (layer_idx < 0 || layer_idx >= kv->num_layers) return fail(AESIR_ERR_INVALID, "KVCache.%s: layer_idx out of bounds", nm);
    if (seq_len <= 0 || seq_len > kv->max_seq) return fail(AESIR_ERR_INVALID, "KVCache.%s: seq_len out of bounds", nm);
    *ptr = (is_k ? kv->k : kv->v) + layer_idx * kv->max_seq * kv->hidden_dim;
    return AESIR_OK;
}

int32_t aesir_kv_k_slice(const aesir_kv *kv, int64_t layer_idx, int64_t seq_len, void **dev_ptr) {
    return kv_slice(kv, layer_idx, seq_len, true, dev_ptr);
}

int32_t aesir_kv_v_slice(const aesir_kv *kv, int64_t layer_idx, int64_t seq_len, void **dev_ptr) {
    return kv_slice(kv, layer_idx, seq_len, false, dev_ptr);
}

}  // extern "C"
