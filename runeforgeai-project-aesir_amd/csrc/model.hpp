// Internal layout of aesir_model (one Llama F16 model in the context's HBM arena).
#pragma once

#include <string>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

namespace aesir {

// Per-layer device tensors. Q, K and V rows are concatenated ([dim + 2 kvd][dim]) so one GEMV
// produces q|k|v; gate and up rows are interleaved (row 2i = gate i, row 2i+1 = up i) so the
// SwiGLU pair of an output lands in one workgroup.
// Q8_0 models store every matrix as int8 quants in the same row order plus f16 block scales
// [rows][cols / 32] (the s* pointers; null for F16 models).
struct ModelLayer {
    void *attn_norm = nullptr;  // [dim]
    void *wqkv = nullptr;       // [dim + 2 kvd][dim]
    void *wo = nullptr;         // [dim][dim]
    void *ffn_norm = nullptr;   // [dim]
    void *wgu = nullptr;        // [2 ffn][dim]
    void *wdown = nullptr;      // [dim][ffn]
    void *sqkv = nullptr, *so = nullptr, *sgu = nullptr, *sdown = nullptr;
    // Q4_0 / Q4_K / Q6_K models: w* hold the nibble records and s* the s0 planes (QFMat); the
    // s1 and hb planes are here (null where the type has none)
    void *qkv_s1 = nullptr, *qkv_hb = nullptr, *o_s1 = nullptr, *o_hb = nullptr;
    void *gu_s1 = nullptr, *gu_hb = nullptr, *down_s1 = nullptr, *down_hb = nullptr;
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
};

}  // namespace aesir

struct aesir_model {
    aesir_ctx *ctx = nullptr;
    aesir_model_config cfg{};
    int64_t hd = 0, kvd = 0;
    float attn_scale = 0.0f, out_eps = 1e-5f;
    int64_t well_start = 0;
    int32_t wtype = AESIR_GGML_F16;  // matrices: AESIR_GGML_F16 or AESIR_GGML_Q8_0
    void *tok_embd = nullptr, *out_norm = nullptr, *out_w = nullptr;
    void *tok_embd_s = nullptr, *out_w_s = nullptr;  // Q8_0 block scales; s0 planes of 4-bit types
    void *tok_embd_s1 = nullptr, *tok_embd_hb = nullptr, *out_w_s1 = nullptr, *out_w_hb = nullptr;
    void *pf_wdeq = nullptr;  // 4-bit types: f16 copy of the matrix a prefill GEMM is reading
    std::vector<aesir::ModelLayer> layers;
    void *k_cache = nullptr, *v_cache = nullptr;  // [n_layers][ctx_len][kvd]
    void *x = nullptr, *q = nullptr, *attn = nullptr, *act = nullptr, *logits = nullptr;
    float *attn_part = nullptr;
    int64_t attn_max_split = 1;
    // batched prefill workspace: pf_rows rows of x, normed x, q|k|v, q, attention out, act,
    // gate/up products (non-MFMA shapes only) and the rows' token IDs
    int64_t pf_rows = 0;
    void *pf_x = nullptr, *pf_xn = nullptr, *pf_qkv = nullptr, *pf_q = nullptr, *pf_att = nullptr, *pf_act = nullptr;
    void *pf_gu = nullptr, *pf_tokens = nullptr;
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
// QFMat of one matrix of a Q4_0 / Q4_K / Q6_K model.
QFMat model_qf(const aesir_model *m, const void *w, const void *s0, const void *s1, const void *hb);
// Batched prefill of tokens[0..n) at positions start_pos.., in chunks of pf_rows rows; *next is the
// greedy token after the last position.
int32_t model_prefill(aesir_model *m, const int64_t *tokens, int64_t n, int64_t start_pos, int64_t *next);
// f32 split-K partial floats the prefill GEMMs of a model with these shapes need at `rows` rows.
int64_t prefill_part_floats(int64_t rows, int64_t dim, int64_t qkv_n, int64_t ffn);
// Decode-step helpers shared with the prefill.
int32_t ensure_rope(aesir_model *m, int64_t max_pos);
int32_t upload_state(aesir_model *m, int64_t token, int64_t pos, int64_t advance, int64_t ring_cap);
LmHeadArgs lm_args(aesir_model *m, bool with_ring);
// One decode step of `token` at `pos` (graph replay when enabled); waits and returns the greedy token.
int32_t model_step(aesir_model *m, int64_t token, int64_t pos, int64_t *next);

}  // namespace aesir
