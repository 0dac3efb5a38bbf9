// Internal layout of aesir_model (one Llama F16 model in the context's HBM arena).
#pragma once

#include <string>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

namespace aesir {

// One device matrix: f16 [rows][cols] (F16); int8 quants [rows][cols] plus f16 block scales
// [rows][cols / 32] in s0 (Q8_0); or the tiled record planes of a 4-bit type (Q4_0 / Q4_K /
// Q6_K: w the nibble plane, s0, s1 and hb as QFMat describes them, null where the type has none).
struct WMat {
    int32_t type = AESIR_GGML_F16;
    void *w = nullptr, *s0 = nullptr, *s1 = nullptr, *hb = nullptr;
};

// Per-layer device tensors. Q, K and V rows are concatenated ([dim + 2 kvd][dim]) so one GEMV
// produces q|k|v; gate and up rows are interleaved (row 2i = gate i, row 2i+1 = up i) so the
// SwiGLU pair of an output lands in one workgroup.
struct ModelLayer {
    void *attn_norm = nullptr;  // [dim]
    void *ffn_norm = nullptr;   // [dim]
    WMat qkv;                   // [dim + 2 kvd][dim], or rows [0, qkv_split) of it
    WMat qkv_b;                 // qkv_split > 0: rows [qkv_split, dim + 2 kvd), in another repacked type
    int64_t qkv_split = 0;
    WMat o;                     // [dim][dim]
    WMat gu;                    // [2 ffn][dim]
    WMat down;                  // [dim][ffn]
};

// GGML types of the model's matrices as the caller uploads them (one per GGUF tensor). A Q/K/V
// matrix whose parts split into two repacked types at a part boundary (Q and K in one type, V in
// another, as the K-quant mixes lay it out; or Q in one, K and V in another) is stored as those
// two parts. Any other fused matrix whose parts differ (Q, K, V; gate, up) is stored as f16, its
// parts dequantized at upload to the f16 weights their own type defines, which are the values
// every path multiplies.
struct LayerTypes {
    int32_t q, k, v, o, gate, up, down;
};
struct WeightTypes {
    int32_t embd = AESIR_GGML_F16, out = AESIR_GGML_F16;
    std::vector<LayerTypes> layers;
};

enum class TensorKind : int {
    TokenEmbd = 0,
    OutputNorm,
    Output,
    AttnNorm,
    AttnQ,
    AttnK,
    AttnV,
    AttnOut,
    FfnNorm,
    FfnGate,
    FfnUp,
    FfnDown
};

struct TensorRef {
    TensorKind kind;
    int layer;  // -1 for global tensors
};

// GGUF shape and device placement: element (r, c) at base + r * row_stride + c (elements of
// esize bytes: 2 for f16, 1 for Q8_0 quants); a Q8_0 matrix's block scale (r, c / 32) at
// scale + r * scale_stride + c / 32 (f16). For Q4_0 / Q4_K / Q6_K matrices (esize 0), row r of
// the tensor is plane row row0 + r * step of the QFMat {qtype, base, hb, scale, s1, row0}.
// in_type is the GGML type the tensor is uploaded as (a quantized part of an f16-stored fused
// matrix is dequantized into it).
struct TensorPlace {
    int64_t rows, cols;
    void *base;
    int64_t row_stride;
    bool is_norm;
    int esize = 2;
    void *scale = nullptr;
    int64_t scale_stride = 0;
    int32_t qtype = 0;
    void *s1 = nullptr, *hb = nullptr;
    int64_t step = 1;
    int64_t row0 = 0;  // 4-bit types: plane row of the tensor's row 0
    int32_t in_type = AESIR_GGML_F16;
};

}  // namespace aesir

struct aesir_model {
    aesir_ctx *ctx = nullptr;
    aesir_model_config cfg{};
    int64_t hd = 0, kvd = 0;
    float attn_scale = 0.0f, out_eps = 1e-5f;
    int64_t well_start = 0;
    // the model's weight type (aesir_model_weight_type): the type of every matrix, or
    // AESIR_WEIGHT_MIXED for a model whose matrices differ
    int32_t wtype = AESIR_GGML_F16;
    aesir::WeightTypes types;  // per GGUF tensor
    bool all_f16 = true;       // every matrix stored as f16
    aesir::WMat embd, out;     // token_embd [vocab][dim], output [vocab][dim]
    void *out_norm = nullptr;
    void *pf_wdeq = nullptr;  // repacked types: f16 copy of the matrix a short-chunk prefill GEMM reads
    std::vector<aesir::ModelLayer> layers;
    void *k_cache = nullptr, *v_cache = nullptr;  // [n_layers][ctx_len][kvd]
    void *x = nullptr, *q = nullptr, *attn = nullptr, *act = nullptr, *logits = nullptr;
    float *attn_part = nullptr;
    int64_t attn_max_split = 1;
    // batched prefill workspace: pf_rows rows of x, normed x, q|k|v, q, attention out, act,
    // gate/up products (non-MFMA shapes, and the library GEMMs' f16 gate/up or f32 residual
    // products) and the rows' token IDs; the library GEMMs' workspace
    int64_t pf_rows = 0;
    void *pf_x = nullptr, *pf_xn = nullptr, *pf_qkv = nullptr, *pf_q = nullptr, *pf_att = nullptr, *pf_act = nullptr;
    void *pf_gu = nullptr, *pf_tokens = nullptr, *pf_blas_ws = nullptr;
    float *pf_part = nullptr;  // f32 split-K partials of the prefill GEMMs
    int64_t pf_part_floats = 0;
    void *lm_parts = nullptr;
    aesir::DecodeState *state = nullptr;  // device
    aesir::DecodeState *state_host = nullptr;  // pinned staging
    int64_t *ring = nullptr;
    int64_t ring_cap = 0;
    const void *rope = nullptr;
    bool use_graph = true;
    bool graph_ready = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
};

namespace aesir {

int32_t parse_tensor_name(const aesir_model *m, const char *name, TensorRef *ref);
TensorPlace place_tensor(const aesir_model *m, const TensorRef &ref);
std::vector<TensorRef> all_tensors(const aesir_model *m);
std::string tensor_name(const TensorRef &ref);
int32_t model_upload(aesir_model *m, const TensorRef &ref, const void *host, int64_t rows, int64_t cols, int32_t type);
// Creates a model whose GGUF tensors have the given types (every matrix type one of F16, Q8_0,
// Q4_0, Q4_K, Q6_K).
int32_t model_create(aesir_ctx *ctx, const aesir_model_config *cfg, const WeightTypes &types, aesir_model **out);
// QFMat of a matrix stored as a Q4_0 / Q4_K / Q6_K type.
QFMat wmat_qf(const WMat &w);
// X[r] = the f16 embedding row tokens[r] of `e` (any matrix type), r < n (tokens on the device).
int32_t launch_embed_rows(hipStream_t s, const WMat &e, int64_t dim, const int64_t *tokens, int64_t n, void *X);
// Batched prefill of tokens[0..n) at positions start_pos.., in chunks of pf_rows rows; *next is the
// greedy token after the last position.
int32_t model_prefill(aesir_model *m, const int64_t *tokens, int64_t n, int64_t start_pos, int64_t *next);
// f32 split-K partial floats the prefill GEMMs of a model with these shapes need for chunks of up
// to `rows` rows.
int64_t prefill_part_floats(int64_t rows, int64_t dim, int64_t qkv_n, int64_t ffn);
// True when every prefill GEMM of this shape runs on the matrix cores (no fallback buffers needed).
bool prefill_gemm_shapes_ok(int64_t rows, int64_t dim, int64_t qkv_n, int64_t ffn);
// Chunk rows from which F16 prefill GEMMs run on hipBLASLt, and the workspace bytes they get.
int64_t prefill_blas_min_rows();
int64_t prefill_blas_workspace();
// Decode-step helpers shared with the prefill.
int32_t ensure_rope(aesir_model *m, int64_t max_pos);
int32_t upload_state(aesir_model *m, int64_t token, int64_t pos, int64_t advance, int64_t ring_cap);
LmHeadArgs lm_args(aesir_model *m, bool with_ring);
// One decode step of `token` at `pos` (graph replay when enabled); waits and returns the greedy token.
int32_t model_step(aesir_model *m, int64_t token, int64_t pos, int64_t *next);

}  // namespace aesir
