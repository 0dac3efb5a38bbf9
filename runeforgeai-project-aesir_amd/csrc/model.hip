// One Llama F16 model resident in the context's HBM arena, its decode step, and the engine loop.
//
// Replaces TransformerBlock.forward / forward_pass (core/inference.mojo:143-275, 424-518) and
// AesirEngine._run_generation (aesir.mojo:323-462). A decode step is 1 + 5 * n_layers + 1 kernel
// launches, all reading the token and position from a device-resident DecodeState, so one
// captured HIP graph replays every step:
//   embed                                x = token_embd[token]
//   per layer  qkv_rope_kv               rmsnorm(x) -> [Q|K|V] GEMV -> RoPE(Q,K) -> K,V into the cache
//              attention                 split-KV GQA over positions [0, min(pos+1, ctx))
//              o + residual              x = f16(f16(Wo attn) + x)
//              gate_up_swiglu            rmsnorm(x) -> [gate,up] GEMV -> f16(up * silu(gate))
//              down + residual           x = f16(f16(Wdown act) + x)
//   lm_head_argmax                       rmsnorm(x) -> logits -> greedy token (-> next step's state)
#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>

#include "common.hpp"
#include "kernels.hpp"
#include "model.hpp"

namespace aesir {

static int32_t carve(aesir_ctx *ctx, int64_t bytes, void **p) { return well_alloc_bytes(ctx, bytes, p); }

// Parses "blk.<l>.<base>.weight" / "<global>.weight" into a tensor id.
int32_t parse_tensor_name(const aesir_model *m, const char *name, TensorRef *ref) {
    std::string s(name ? name : "");
    const std::string suffix = ".weight";
    if (s.size() <= suffix.size() || s.compare(s.size() - suffix.size(), suffix.size(), suffix) != 0)
        return fail(AESIR_ERR_FORMAT, "GGUF tensor name is not a weight: %s", s.c_str());
    std::string stem = s.substr(0, s.size() - suffix.size());
    ref->layer = -1;
    if (stem == "token_embd") {
        ref->kind = TensorKind::TokenEmbd;
        return AESIR_OK;
    }
    if (stem == "output_norm") {
        ref->kind = TensorKind::OutputNorm;
        return AESIR_OK;
    }
    if (stem == "output") {
        ref->kind = TensorKind::Output;
        return AESIR_OK;
    }
    if (stem.rfind("blk.", 0) == 0) {
        size_t dot = stem.find('.', 4);
        if (dot == std::string::npos) return fail(AESIR_ERR_FORMAT, "GGUF tensor name is malformed: %s", s.c_str());
        char *end = nullptr;
        long layer = std::strtol(stem.c_str() + 4, &end, 10);
        if (end != stem.c_str() + dot || layer < 0 || layer >= m->cfg.n_layers)
            return fail(AESIR_ERR_FORMAT, "GGUF tensor layer index out of range: %s", s.c_str());
        std::string base = stem.substr(dot + 1);
        static const struct {
            const char *n;
            TensorKind k;
        } table[] = {{"attn_norm", TensorKind::AttnNorm}, {"attn_q", TensorKind::AttnQ},
                     {"attn_k", TensorKind::AttnK},       {"attn_v", TensorKind::AttnV},
                     {"attn_output", TensorKind::AttnOut}, {"ffn_norm", TensorKind::FfnNorm},
                     {"ffn_gate", TensorKind::FfnGate},   {"ffn_up", TensorKind::FfnUp},
                     {"ffn_down", TensorKind::FfnDown}};
        for (auto &t : table) {
            if (base == t.n) {
                ref->kind = t.k;
                ref->layer = (int)layer;
                return AESIR_OK;
            }
        }
    }
    return fail(AESIR_ERR_FORMAT, "GGUF tensor is not part of the Llama F16 path: %s", s.c_str());
}

// Expected GGUF shape (rows, cols) and the device placement of a tensor: element (r, c) of the
// GGUF tensor lives at base + r * row_stride + c (and its Q8_0 block scale at
// scale + r * scale_stride + c / 32); a 4-bit tensor's row r is plane row row0 + r * step.
TensorPlace place_tensor(const aesir_model *m, const TensorRef &ref) {
    const int64_t d = m->cfg.dim, kvd = m->kvd, f = m->cfg.ffn, V = m->cfg.vocab;
    const ModelLayer *L = ref.layer >= 0 ? &m->layers[ref.layer] : nullptr;
    const LayerTypes *T = ref.layer >= 0 ? &m->types.layers[ref.layer] : nullptr;
    // matrix rows [r0, r0 + rows) of a fused matrix w with `cols` columns, every `step`-th row,
    // uploaded as in_type
    auto mat = [&](int64_t rows, int64_t cols, const WMat &w, int64_t r0, int64_t step, int32_t in_type) {
        if (qf_type(w.type)) {
            TensorPlace p{rows, cols, w.w, 0, false, 0, w.s0, 0};
            p.qtype = w.type;
            p.s1 = w.s1;
            p.hb = w.hb;
            p.step = step;
            p.row0 = r0;
            p.in_type = in_type;
            return p;
        }
        const bool q8 = w.type == AESIR_GGML_Q8_0;
        const int es = q8 ? 1 : 2;
        TensorPlace p{rows, cols, (char *)w.w + r0 * cols * es, step * cols, false, es, nullptr, 0};
        p.qtype = w.type;
        p.in_type = in_type;
        if (q8) {
            p.scale = (uint16_t *)w.s0 + r0 * (cols / 32);
            p.scale_stride = step * (cols / 32);
        }
        return p;
    };
    auto norm = [&](void *base) { return TensorPlace{1, d, base, d, true, 2, nullptr, 0}; };
    // rows [r0, r0 + rows) of the Q/K/V matrix: in its second part from L->qkv_split on
    auto qkv_part = [&](int64_t r0, int64_t rows, int32_t in_type) {
        if (L->qkv_split > 0 && r0 >= L->qkv_split) return mat(rows, d, L->qkv_b, r0 - L->qkv_split, 1, in_type);
        return mat(rows, d, L->qkv, r0, 1, in_type);
    };
    switch (ref.kind) {
        case TensorKind::TokenEmbd: return mat(V, d, m->embd, 0, 1, m->types.embd);
        case TensorKind::OutputNorm: return norm(m->out_norm);
        case TensorKind::Output: return mat(V, d, m->out, 0, 1, m->types.out);
        case TensorKind::AttnNorm: return norm(L->attn_norm);
        case TensorKind::AttnQ: return qkv_part(0, d, T->q);
        case TensorKind::AttnK: return qkv_part(d, kvd, T->k);
        case TensorKind::AttnV: return qkv_part(d + kvd, kvd, T->v);
        case TensorKind::AttnOut: return mat(d, d, L->o, 0, 1, T->o);
        case TensorKind::FfnNorm: return norm(L->ffn_norm);
        case TensorKind::FfnGate: return mat(f, d, L->gu, 0, 2, T->gate);  // gate i -> fused row 2i
        case TensorKind::FfnUp: return mat(f, d, L->gu, 1, 2, T->up);      // up i -> fused row 2i + 1
        case TensorKind::FfnDown: return mat(d, f, L->down, 0, 1, T->down);
    }
    return TensorPlace{};
}

QFMat wmat_qf(const WMat &w) {
    QFMat q;
    q.type = w.type;
    q.nib = w.w;
    q.s0 = w.s0;
    q.s1 = w.s1;
    q.hb = w.hb;
    return q;
}

static QFMat place_qf(const TensorPlace &p) {
    QFMat q;
    q.type = p.qtype;
    q.nib = p.base;
    q.s0 = p.scale;
    q.s1 = p.s1;
    q.hb = p.hb;
    q.row0 = p.row0;
    return q;
}

static int64_t stream_id(const TensorRef &ref) {
    // Same numbering as the test oracle's generator: globals 0..2, then 100 + 16 * layer + slot.
    switch (ref.kind) {
        case TensorKind::TokenEmbd: return 0;
        case TensorKind::OutputNorm: return 1;
        case TensorKind::Output: return 2;
        default: break;
    }
    int slot = 0;
    switch (ref.kind) {
        case TensorKind::AttnNorm: slot = 0; break;
        case TensorKind::AttnQ: slot = 1; break;
        case TensorKind::AttnK: slot = 2; break;
        case TensorKind::AttnV: slot = 3; break;
        case TensorKind::AttnOut: slot = 4; break;
        case TensorKind::FfnNorm: slot = 5; break;
        case TensorKind::FfnGate: slot = 6; break;
        case TensorKind::FfnUp: slot = 7; break;
        case TensorKind::FfnDown: slot = 8; break;
        default: break;
    }
    return 100 + 16 * ref.layer + slot;
}

std::vector<TensorRef> all_tensors(const aesir_model *m) {
    std::vector<TensorRef> v;
    v.push_back({TensorKind::TokenEmbd, -1});
    v.push_back({TensorKind::OutputNorm, -1});
    v.push_back({TensorKind::Output, -1});
    const TensorKind per[] = {TensorKind::AttnNorm, TensorKind::AttnQ,   TensorKind::AttnK,
                              TensorKind::AttnV,    TensorKind::AttnOut, TensorKind::FfnNorm,
                              TensorKind::FfnGate,  TensorKind::FfnUp,   TensorKind::FfnDown};
    for (int l = 0; l < m->cfg.n_layers; l++)
        for (auto k : per) v.push_back({k, l});
    return v;
}

std::string tensor_name(const TensorRef &ref) {
    static const char *names[] = {"token_embd", "output_norm", "output",   "attn_norm", "attn_q", "attn_k",
                                  "attn_v",     "attn_output", "ffn_norm", "ffn_gate",  "ffn_up", "ffn_down"};
    std::string base = names[(int)ref.kind];
    if (ref.layer >= 0) return "blk." + std::to_string(ref.layer) + "." + base + ".weight";
    return base + ".weight";
}

int32_t model_upload(aesir_model *m, const TensorRef &ref, const void *host, int64_t rows, int64_t cols, int32_t type) {
    const TensorPlace p = place_tensor(m, ref);
    const std::string nm = tensor_name(ref);
    if (rows != p.rows || cols != p.cols)
        return fail(AESIR_ERR_FORMAT, "GGUF required tensor has an invalid shape: %s", nm.c_str());
    hipStream_t s = m->ctx->stream;
    if (!p.is_norm && type != p.in_type)
        return fail(AESIR_ERR_FORMAT, "GGUF required tensor has an invalid type: %s", nm.c_str());
    if (p.esize == 2 && !p.is_norm && type != AESIR_GGML_F16) {
        // a quantized part of an f16-stored fused matrix: its f16 weights, dequantized on the device
        const int64_t bytes = ggml_tensor_bytes(type, rows, cols);
        if (bytes <= 0) return fail(AESIR_ERR_FORMAT, "GGUF required tensor has an invalid shape: %s", nm.c_str());
        void *staging = nullptr;
        AESIR_HIP_TRY(hipMalloc(&staging, (size_t)bytes));
        int32_t rc = AESIR_OK;
        if (hipMemcpyAsync(staging, host, (size_t)bytes, hipMemcpyHostToDevice, s) != hipSuccess)
            rc = fail(AESIR_ERR_HIP, "hipMemcpyAsync of %s failed", nm.c_str());
        if (rc == AESIR_OK) rc = launch_gguf_dequant(s, type, staging, rows, cols, p.base, p.row_stride);
        if (hipStreamSynchronize(s) != hipSuccess && rc == AESIR_OK)
            rc = fail(AESIR_ERR_HIP, "dequantization of %s failed", nm.c_str());
        (void)hipFree(staging);
        return rc;
    }
    if (p.esize == 0) {  // Q4_0 / Q4_K / Q6_K matrix: repack the GGUF blocks on the device
        const int64_t bytes = ggml_tensor_bytes(type, rows, cols);
        if (bytes <= 0) return fail(AESIR_ERR_FORMAT, "GGUF required tensor has an invalid shape: %s", nm.c_str());
        void *staging = nullptr;
        AESIR_HIP_TRY(hipMalloc(&staging, (size_t)bytes));
        int32_t rc = AESIR_OK;
        if (hipMemcpyAsync(staging, host, (size_t)bytes, hipMemcpyHostToDevice, s) != hipSuccess)
            rc = fail(AESIR_ERR_HIP, "hipMemcpyAsync of %s failed", nm.c_str());
        if (rc == AESIR_OK) rc = launch_qf_repack(s, type, staging, rows, cols, place_qf(p), p.step);
        if (hipStreamSynchronize(s) != hipSuccess && rc == AESIR_OK) rc = fail(AESIR_ERR_HIP, "repack of %s failed", nm.c_str());
        (void)hipFree(staging);
        return rc;
    }
    if (p.esize == 1) {  // Q8_0 matrix: split the 34-byte blocks into quants and scales
        const int64_t nb = cols / 32;
        std::vector<int8_t> qs((size_t)(rows * cols));
        std::vector<uint16_t> ds((size_t)(rows * nb));
        const uint8_t *b = (const uint8_t *)host;
        for (int64_t i = 0; i < rows * nb; i++, b += 34) {
            std::memcpy(&ds[i], b, 2);
            std::memcpy(&qs[i * 32], b + 2, 32);
        }
        AESIR_HIP_TRY(hipMemcpy2DAsync(p.base, (size_t)p.row_stride, qs.data(), (size_t)cols, (size_t)cols, (size_t)rows,
                                       hipMemcpyHostToDevice, s));
        AESIR_HIP_TRY(hipMemcpy2DAsync(p.scale, (size_t)p.scale_stride * 2, ds.data(), (size_t)nb * 2, (size_t)nb * 2,
                                       (size_t)rows, hipMemcpyHostToDevice, s));
        AESIR_HIP_TRY(hipStreamSynchronize(s));
        return AESIR_OK;
    }
    if (type != AESIR_GGML_F16 && !(p.is_norm && type == AESIR_GGML_F32))
        return fail(AESIR_ERR_FORMAT, "GGUF required tensor has an invalid type: %s", nm.c_str());
    std::vector<uint16_t> conv;
    const void *src = host;
    if (type == AESIR_GGML_F32) {  // loader/gguf.mojo:486-493: F32 -> f16 (round to nearest even)
        conv.resize((size_t)(rows * cols));
        const float *f = (const float *)host;
        for (int64_t i = 0; i < rows * cols; i++) conv[i] = f32_to_f16_bits(f[i]);
        src = conv.data();
    }
    AESIR_HIP_TRY(hipMemcpy2DAsync(p.base, (size_t)p.row_stride * 2, src, (size_t)cols * 2, (size_t)cols * 2,
                                   (size_t)rows, hipMemcpyHostToDevice, s));
    AESIR_HIP_TRY(hipStreamSynchronize(s));
    return AESIR_OK;
}

// ------------------------------------------------------------------ decode step

// The layer-0 QKV GEMV performs the embedding lookup when the table has the QKV matrix's type;
// otherwise the decode step looks the row up first (embed_lookup).
static bool embd_fused(const aesir_model *m) {
    return m->embd.type == m->layers[0].qkv.type && m->layers[0].qkv_split == 0;
}

static QkvArgs qkv_args(aesir_model *m, int64_t l) {
    const aesir_model_config &c = m->cfg;
    const ModelLayer &L = m->layers[l];
    const bool emb = l == 0 && embd_fused(m);
    QkvArgs a{m->x, emb ? m->embd.w : nullptr, L.attn_norm, c.rms_eps, L.qkv.w, c.dim, m->kvd, m->hd, m->q,
              (uint16_t *)m->k_cache + l * c.ctx_len * m->kvd, (uint16_t *)m->v_cache + l * c.ctx_len * m->kvd,
              c.ctx_len, m->rope, m->state, L.qkv.type == AESIR_GGML_Q8_0 ? L.qkv.s0 : nullptr,
              emb && m->embd.type == AESIR_GGML_Q8_0 ? m->embd.s0 : nullptr};
    if (qf_type(L.qkv.type)) {
        a.wq = wmat_qf(L.qkv);
        if (emb) a.eq = wmat_qf(m->embd);
        if (L.qkv_split > 0) {
            a.qkv_split = L.qkv_split;
            a.wq_b = wmat_qf(L.qkv_b);
        }
    }
    return a;
}

static int32_t embed_lookup(aesir_model *m, hipStream_t s) {
    return launch_embed_rows(s, m->embd, m->cfg.dim, &m->state->token, 1, m->x);
}

// O and down projections with the residual add, and the gate/up GEMV with SwiGLU, for every
// weight type.
static const void *q8_scales(const WMat &w) { return w.type == AESIR_GGML_Q8_0 ? w.s0 : nullptr; }
static int32_t launch_o_residual(aesir_model *m, hipStream_t s, const ModelLayer &L) {
    const int64_t d = m->cfg.dim;
    if (qf_type(L.o.type)) return launch_qf_gemv_residual(s, wmat_qf(L.o), d, d, m->attn, m->x);
    return launch_gemv_residual(s, L.o.w, d, d, m->attn, m->x, q8_scales(L.o));
}
static int32_t launch_down_residual(aesir_model *m, hipStream_t s, const ModelLayer &L) {
    const int64_t d = m->cfg.dim, f = m->cfg.ffn;
    if (qf_type(L.down.type)) return launch_qf_gemv_residual(s, wmat_qf(L.down), d, f, m->act, m->x);
    return launch_gemv_residual(s, L.down.w, d, f, m->act, m->x, q8_scales(L.down));
}
static int32_t launch_gate_up(aesir_model *m, hipStream_t s, const ModelLayer &L) {
    const aesir_model_config &c = m->cfg;
    if (qf_type(L.gu.type))
        return launch_qf_gate_up_swiglu(s, m->x, L.ffn_norm, c.rms_eps, wmat_qf(L.gu), c.ffn, c.dim, m->act);
    return launch_gate_up_swiglu(s, m->x, L.ffn_norm, c.rms_eps, L.gu.w, c.ffn, c.dim, m->act, q8_scales(L.gu));
}

static AttnArgs attn_args(aesir_model *m, int64_t l) {
    const aesir_model_config &c = m->cfg;
    AttnArgs a{};
    a.q = m->q;
    a.k = (uint16_t *)m->k_cache + l * c.ctx_len * m->kvd;
    a.v = (uint16_t *)m->v_cache + l * c.ctx_len * m->kvd;
    a.k_stride = m->kvd;
    a.v_stride = m->kvd;
    a.out = m->attn;
    a.nq = c.n_heads;
    a.nkv = c.n_kv_heads;
    a.hd = m->hd;
    a.scale = m->attn_scale;
    a.seq_len = 0;  // S = min(pos + 1, ctx_len) from the device state
    a.state = m->state;
    a.max_seq = c.ctx_len;
    a.part = m->attn_part;
    a.max_split = m->attn_max_split;
    return a;
}

LmHeadArgs lm_args(aesir_model *m, bool with_ring) {
    const aesir_model_config &c = m->cfg;
    LmHeadArgs a{m->x, m->out_norm, m->out_eps, m->out.w, c.vocab, c.dim, m->logits, m->lm_parts, m->state,
                 with_ring ? m->ring : nullptr, q8_scales(m->out)};
    if (qf_type(m->out.type)) a.wq = wmat_qf(m->out);
    return a;
}

static int32_t enqueue_step(aesir_model *m, hipStream_t s) {
    const aesir_model_config &c = m->cfg;
    const int64_t d = c.dim;
    if (!embd_fused(m)) AESIR_TRY(embed_lookup(m, s));
    for (int64_t l = 0; l < c.n_layers; l++) {
        const ModelLayer &L = m->layers[l];
        AESIR_TRY(launch_qkv_rope_kv(s, qkv_args(m, l)));  // layer 0 may also perform the embedding lookup
        AESIR_TRY(launch_attention_decode(s, attn_args(m, l)));
        AESIR_TRY(launch_o_residual(m, s, L));
        AESIR_TRY(launch_gate_up(m, s, L));
        AESIR_TRY(launch_down_residual(m, s, L));
    }
    return launch_lm_head_argmax(s, lm_args(m, true));
}

int32_t ensure_rope(aesir_model *m, int64_t max_pos) {
    const void *t = nullptr;
    AESIR_TRY(rope_table(m->ctx, m->cfg.rope_theta, m->hd, max_pos, &t));
    if (t != m->rope) {
        m->rope = t;
        if (m->graph_ready) {  // the table pointer is baked into the captured graph
            (void)hipGraphExecDestroy(m->graph_exec);
            (void)hipGraphDestroy(m->graph);
            m->graph_ready = false;
        }
    }
    return AESIR_OK;
}

static int32_t ensure_graph(aesir_model *m) {
    if (m->graph_ready || !m->use_graph) return AESIR_OK;
    hipStream_t s = m->ctx->stream;
    AESIR_HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int32_t rc = enqueue_step(m, s);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(s, &g);
    if (rc != AESIR_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return fail(AESIR_ERR_HIP, "hipStreamEndCapture failed: %s", hipGetErrorString(e));
    e = hipGraphInstantiate(&m->graph_exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return fail(AESIR_ERR_HIP, "hipGraphInstantiate failed: %s", hipGetErrorString(e));
    }
    m->graph = g;
    m->graph_ready = true;
    return AESIR_OK;
}

static int32_t run_step(aesir_model *m, bool graph) {
    hipStream_t s = m->ctx->stream;
    if (graph && m->use_graph) {
        AESIR_TRY(ensure_graph(m));
        AESIR_HIP_TRY(hipGraphLaunch(m->graph_exec, s));
        return AESIR_OK;
    }
    return enqueue_step(m, s);
}

int32_t model_step(aesir_model *m, int64_t token, int64_t pos, int64_t *next) {
    AESIR_TRY(upload_state(m, token, pos, 0, m->ring_cap));
    AESIR_TRY(run_step(m, true));
    AESIR_HIP_TRY(hipMemcpyAsync(m->state_host, m->state, sizeof(DecodeState), hipMemcpyDeviceToHost, m->ctx->stream));
    AESIR_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    *next = m->state_host->next_token;
    return AESIR_OK;
}

int32_t upload_state(aesir_model *m, int64_t token, int64_t pos, int64_t advance, int64_t ring_cap) {
    DecodeState *h = m->state_host;
    std::memset(h, 0, sizeof(DecodeState));
    h->token = token;
    h->pos = pos;
    h->next_token = 0;
    h->step = 0;
    h->advance = advance;
    h->ring_cap = ring_cap;
    AESIR_HIP_TRY(hipMemcpyAsync(m->state, h, sizeof(DecodeState), hipMemcpyHostToDevice, m->ctx->stream));
    return AESIR_OK;
}

}  // namespace aesir

using namespace aesir;

extern "C" {

int32_t aesir_model_create(aesir_ctx *ctx, const aesir_model_config *cfg, aesir_model **out) {
    return aesir_model_create_typed(ctx, cfg, AESIR_GGML_F16, out);
}

int32_t aesir_model_weight_type(const aesir_model *m) { return m ? m->wtype : -1; }

int32_t aesir_model_create_typed(aesir_ctx *ctx, const aesir_model_config *cfg, int32_t weight_type,
                                 aesir_model **out) {
    WeightTypes t;
    t.embd = t.out = weight_type;
    if (cfg && cfg->n_layers > 0 && cfg->n_layers <= ((int64_t)1 << 31))
        t.layers.assign((size_t)cfg->n_layers, LayerTypes{weight_type, weight_type, weight_type, weight_type,
                                                          weight_type, weight_type, weight_type});
    return model_create(ctx, cfg, t, out);
}

int32_t aesir_model_create_mixed(aesir_ctx *ctx, const aesir_model_config *cfg, const int32_t *tensor_types,
                                 int64_t n_types, aesir_model **out) {
    if (!cfg || !tensor_types || !out) return fail(AESIR_ERR_INVALID, "aesir_model_create_mixed: null argument");
    if (cfg->n_layers <= 0 || cfg->n_layers > ((int64_t)1 << 31) || n_types != 2 + 7 * cfg->n_layers)
        return fail(AESIR_ERR_INVALID, "aesir_model_create_mixed: need 2 + 7 * n_layers tensor types");
    WeightTypes t;
    t.embd = tensor_types[0];
    t.out = tensor_types[1];
    t.layers.resize((size_t)cfg->n_layers);
    for (int64_t l = 0; l < cfg->n_layers; l++) {
        const int32_t *v = tensor_types + 2 + 7 * l;
        t.layers[l] = LayerTypes{v[0], v[1], v[2], v[3], v[4], v[5], v[6]};
    }
    return model_create(ctx, cfg, t, out);
}

int32_t aesir_model_tensor_type(aesir_model *m, const char *name) {
    if (!m || !name) return fail(AESIR_ERR_INVALID, "aesir_model_tensor_type: null argument");
    TensorRef ref;
    AESIR_TRY(parse_tensor_name(m, name, &ref));
    return place_tensor(m, ref).in_type;
}

}  // extern "C"

namespace aesir {

// Types a matrix keeps in HBM as they are (the others are stored in f16).
static bool stored_native(int32_t t) { return t == AESIR_GGML_F16 || t == AESIR_GGML_Q8_0 || qf_type(t); }

int32_t model_create(aesir_ctx *ctx, const aesir_model_config *cfg, const WeightTypes &types, aesir_model **out) {
    AESIR_TRY(bind(ctx));
    if (!cfg || !out) return fail(AESIR_ERR_INVALID, "aesir_model_create: null argument");
    *out = nullptr;
    const aesir_model_config c = *cfg;
    // GGUFModelConfig.validate (loader/gguf.mojo:133-149)
    if (c.ctx_len <= 0 || c.dim <= 0) return fail(AESIR_ERR_FORMAT, "GGUF model dimensions are incomplete");
    if (c.ffn <= 0 || c.n_layers <= 0) return fail(AESIR_ERR_FORMAT, "GGUF layer metadata is incomplete");
    if (c.n_heads <= 0 || c.n_kv_heads <= 0) return fail(AESIR_ERR_FORMAT, "GGUF attention metadata is incomplete");
    if (c.dim % c.n_heads != 0) return fail(AESIR_ERR_FORMAT, "GGUF embedding length is not divisible by head count");
    if (c.n_heads % c.n_kv_heads != 0) return fail(AESIR_ERR_FORMAT, "GGUF query heads are not divisible by KV heads");
    if (c.vocab <= 0) return fail(AESIR_ERR_FORMAT, "GGUF vocabulary is empty");
    // Dimensions up to 2^31 keep every sum below exact; every product is checked where it is formed.
    const int64_t lim = (int64_t)1 << 31;
    if (c.dim > lim || c.ffn > lim || c.vocab > lim || c.ctx_len > lim || c.n_layers > lim)
        return fail(AESIR_ERR_FORMAT, "model: a dimension exceeds 2^31");
    if (!(c.rms_eps > 0.0f)) return fail(AESIR_ERR_INVALID, "rmsnorm: epsilon must be positive");
    const int64_t hd = c.dim / c.n_heads;
    if (hd % 2 != 0) return fail(AESIR_ERR_INVALID, "apply_rope: head_dim must be positive and even");
    if (hd > 256 || c.n_heads / c.n_kv_heads > 16)
        return fail(AESIR_ERR_UNSUPPORTED, "model: head_dim <= 256 and <= 16 query heads per KV head are supported");
    if ((int64_t)types.layers.size() != c.n_layers)
        return fail(AESIR_ERR_INVALID, "model: one set of weight types per layer is needed");
    // every matrix type present, each checked once against dim and ffn
    std::vector<int32_t> present{types.embd, types.out};
    for (const LayerTypes &t : types.layers)
        for (int32_t v : {t.q, t.k, t.v, t.o, t.gate, t.up, t.down}) present.push_back(v);
    std::sort(present.begin(), present.end());
    present.erase(std::unique(present.begin(), present.end()), present.end());
    for (int32_t wt : present) {
        if (wt != AESIR_GGML_F16 && gguf_block_elems(wt) == 0)
            return fail(AESIR_ERR_UNSUPPORTED,
                        "model: weight type %d is not F16, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q4_K, Q5_K or Q6_K",
                        (int)wt);
        if (!stored_native(wt)) {
            // kept in f16, dequantized at upload: whole blocks per row
            const int64_t blk = gguf_block_elems(wt);
            if (c.dim % blk != 0 || c.ffn % blk != 0)
                return fail(AESIR_ERR_UNSUPPORTED, "model: %s weights need dim and ffn to be multiples of %lld",
                            ggml_type_name(wt), (long long)blk);
        }
        if (wt == AESIR_GGML_Q8_0 && (c.dim % 32 != 0 || c.ffn % 32 != 0 || c.dim > kQ8GemvMaxK || c.ffn > kQ8GemvMaxK))
            return fail(AESIR_ERR_UNSUPPORTED, "model: Q8_0 weights need dim and ffn to be multiples of 32, at most 28672");
        if (qf_type(wt)) {
            // whole 128-weight segments of the repacked planes; K-quant super-blocks of 256
            const int64_t blk = gguf_block_elems(wt) == 32 ? 128 : 256;
            if (c.dim % blk != 0 || c.ffn % blk != 0 || c.dim > kQfGemvMaxK || c.ffn > kQfGemvMaxK)
                return fail(AESIR_ERR_UNSUPPORTED,
                            "model: %s weights need dim and ffn to be multiples of %lld, at most 28672",
                            ggml_type_name(wt), (long long)blk);
        }
    }

    auto *m = new aesir_model();
    m->ctx = ctx;
    m->cfg = c;
    m->types = types;
    // the stored model type: the matrices' common type, else AESIR_WEIGHT_MIXED
    m->wtype = present.size() == 1 ? present[0] : AESIR_WEIGHT_MIXED;
    m->hd = hd;
    m->kvd = hd * c.n_kv_heads;
    m->attn_scale = (float)(1.0 / std::pow((double)hd, 0.5));  // compute.mojo:1968
    m->out_eps = c.rms_eps > 0.0f ? c.rms_eps : 1e-5f;           // inference.mojo:484-488
    m->well_start = ctx->well_offset;
    const int64_t d = c.dim, kvd = m->kvd, f = c.ffn, V = c.vocab;
    auto fail_cleanup = [&](int32_t rc) {
        ctx->well_offset = m->well_start;
        delete m;
        return rc;
    };
    int32_t rc = AESIR_OK;
    // Every size below is a checked product (mul_checked is -1 on overflow): a config read from
    // a file must not wrap into a small allocation.
    auto take = [&](int64_t bytes, void **p) {
        if (rc == AESIR_OK && bytes < 0) rc = fail(AESIR_ERR_FORMAT, "model: a tensor size overflows int64");
        if (rc == AESIR_OK) rc = carve(ctx, bytes, p);
    };
    // a matrix of rows x cols stored as `type`: f16, int8 quants plus f16 block scales (Q8_0), or
    // the record planes of a 4-bit type (nibbles, then s0, s1 and hb where the type has them)
    bool any_qf = false;
    auto matrix = [&](int64_t rows, int64_t cols, int32_t type, WMat *w) {
        w->type = type;
        if (qf_type(type)) {
            any_qf = true;
            for (int plane = 0; plane < 4; plane++) {
                const int64_t rb = qf_plane_row_bytes(type, plane, cols);
                if (rb > 0)
                    take(mul_checked(qf_rows_alloc(rows), rb), plane == 0 ? &w->w : plane == 1 ? &w->hb : plane == 2 ? &w->s0 : &w->s1);
            }
            return;
        }
        const bool q8 = type == AESIR_GGML_Q8_0;
        take(mul_checked(rows, cols, q8 ? 1 : 2), &w->w);
        if (q8) take(mul_checked(rows, cols / 32, 2), &w->s0);
    };
    // A fused matrix whose parts differ in type is stored in f16 (each part dequantized at upload),
    // as is every matrix of a type without a GEMV of its own.
    auto fused = [](std::initializer_list<int32_t> parts) {
        const int32_t t0 = *parts.begin();
        for (int32_t t : parts)
            if (t != t0) return (int32_t)AESIR_GGML_F16;
        return stored_native(t0) ? t0 : (int32_t)AESIR_GGML_F16;
    };
    matrix(V, d, fused({types.embd}), &m->embd);
    take(d * 2, &m->out_norm);
    matrix(V, d, fused({types.out}), &m->out);
    m->layers.resize((size_t)c.n_layers);
    for (int64_t l = 0; l < c.n_layers; l++) {
        ModelLayer &L = m->layers[l];
        const LayerTypes &t = types.layers[l];
        take(d * 2, &L.attn_norm);
        // Q/K/V in two repacked types split at a part boundary: two parts, one two-part GEMV
        int64_t split = 0;
        if (t.q == t.k && t.k != t.v && qf_type(t.q) && qf_type(t.v) && qf_qkv_pair_ok(t.q, t.v)) split = d + kvd;
        if (t.q != t.k && t.k == t.v && qf_type(t.q) && qf_type(t.k) && qf_qkv_pair_ok(t.q, t.k)) split = d;
        if (split > 0 && split % 16 == 0 && kvd % 16 == 0) {
            matrix(split, d, t.q, &L.qkv);
            matrix(d + 2 * kvd - split, d, t.v, &L.qkv_b);
            L.qkv_split = split;
        } else {
            matrix(d + 2 * kvd, d, fused({t.q, t.k, t.v}), &L.qkv);
        }
        matrix(d, d, fused({t.o}), &L.o);
        take(d * 2, &L.ffn_norm);
        matrix(2 * f, d, fused({t.gate, t.up}), &L.gu);
        matrix(d, f, fused({t.down}), &L.down);
    }
    m->all_f16 = m->embd.type == AESIR_GGML_F16 && m->out.type == AESIR_GGML_F16;
    for (const ModelLayer &L : m->layers)
        for (const WMat *w : {&L.qkv, &L.o, &L.gu, &L.down}) m->all_f16 = m->all_f16 && w->type == AESIR_GGML_F16;
    // f16 copy of the largest layer matrix for the prefill GEMMs: repacked types dequantize into it
    // for short chunks off the wide tile, and every quantized matrix for the library GEMMs of long
    // chunks (Q8_0 only then)
    const int64_t pr_max = c.ctx_len < 2048 ? c.ctx_len : 2048;
    bool q8_mats = false;
    for (const ModelLayer &L : m->layers)
        for (const WMat *w : {&L.qkv, &L.qkv_b, &L.o, &L.gu, &L.down}) q8_mats = q8_mats || w->type == AESIR_GGML_Q8_0;
    if (any_qf || (q8_mats && pr_max >= prefill_blas_min_rows())) {
        int64_t big = (d + 2 * kvd) * d;
        if (2 * f * d > big) big = 2 * f * d;
        take(mul_checked(big, 2), &m->pf_wdeq);
    }
    take(mul_checked(c.n_layers, c.ctx_len, kvd, 2), &m->k_cache);
    take(mul_checked(c.n_layers, c.ctx_len, kvd, 2), &m->v_cache);
    take(d * 2, &m->x);
    take(d * 2, &m->q);
    take(d * 2, &m->attn);
    take(f * 2, &m->act);
    take(V * 2, &m->logits);
    const int64_t max_split = attention_split_count(hd, c.ctx_len);
    m->attn_max_split = max_split;
    void *p = nullptr;
    take(attention_partial_floats(c.n_heads, hd, max_split) * 4, &p);
    m->attn_part = (float *)p;
    take(lm_head_groups(V) * 8, &m->lm_parts);
    m->pf_rows = c.ctx_len < 2048 ? c.ctx_len : 2048;  // batched-prefill chunk
    const int64_t pr = m->pf_rows;
    take(pr * d * 2, &m->pf_x);
    take(pr * d * 2, &m->pf_xn);
    take(pr * (d + 2 * kvd) * 2, &m->pf_qkv);
    take(pr * d * 2, &m->pf_q);
    take(pr * d * 2, &m->pf_att);
    take(pr * f * 2, &m->pf_act);
    // chunks of many rows run their GEMMs on hipBLASLt (quantized matrices through the f16 copy in
    // pf_wdeq), whose gate/up (f16) and residual (f32) products pass through pf_gu
    const bool blas = pr >= prefill_blas_min_rows();
    if (!prefill_gemm_shapes_ok(pr, d, d + 2 * kvd, f) || blas)
        take(pr * 2 * f * 2 > pr * d * 4 ? pr * 2 * f * 2 : pr * d * 4, &m->pf_gu);
    if (blas) take(prefill_blas_workspace(), &m->pf_blas_ws);
    take(pr * 8, &m->pf_tokens);
    m->pf_part_floats = prefill_part_floats(pr, d, d + 2 * kvd, f);
    if (m->pf_part_floats > 0) {
        take(m->pf_part_floats * 4, &p);
        m->pf_part = (float *)p;
    }
    take(sizeof(DecodeState), &p);
    m->state = (DecodeState *)p;
    m->ring_cap = 65536;
    take(m->ring_cap * 8, &p);
    m->ring = (int64_t *)p;
    if (rc != AESIR_OK) return fail_cleanup(rc);
    // The well may hold an earlier model's bytes: clear the whole model region.
    const int64_t used = (ctx->well_offset - m->well_start) * 2;
    if (hipMemsetAsync(ctx->well_base + m->well_start * 2, 0, (size_t)used, ctx->stream) != hipSuccess)
        return fail_cleanup(fail(AESIR_ERR_HIP, "hipMemsetAsync of the model region failed"));
    if (hipHostMalloc((void **)&m->state_host, sizeof(DecodeState), hipHostMallocDefault) != hipSuccess)
        return fail_cleanup(fail(AESIR_ERR_HIP, "hipHostMalloc failed"));
    m->use_graph = true;
    if (const char *e = std::getenv("AESIR_NO_GRAPH")) m->use_graph = e[0] == '0';
    if ((rc = ensure_rope(m, c.ctx_len)) != AESIR_OK) return fail_cleanup(rc);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return fail_cleanup(fail(AESIR_ERR_HIP, "sync failed"));
    ctx->live_models++;
    *out = m;
    return AESIR_OK;
}

}  // namespace aesir

extern "C" {

int32_t aesir_model_destroy(aesir_model *m) {
    if (!m) return AESIR_OK;
    (void)hipSetDevice(m->ctx->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    if (m->graph_ready) {
        (void)hipGraphExecDestroy(m->graph_exec);
        (void)hipGraphDestroy(m->graph);
    }
    if (m->state_host) (void)hipHostFree(m->state_host);
    m->ctx->live_models--;
    delete m;
    return AESIR_OK;
}

int32_t aesir_model_get_config(const aesir_model *m, aesir_model_config *cfg) {
    if (!m || !cfg) return fail(AESIR_ERR_INVALID, "aesir_model_get_config: null argument");
    *cfg = m->cfg;
    return AESIR_OK;
}

int32_t aesir_model_set_tensor(aesir_model *m, const char *name, const void *host_data, int64_t rows, int64_t cols,
                               int32_t ggml_type) {
    if (!m || !host_data) return fail(AESIR_ERR_INVALID, "aesir_model_set_tensor: null argument");
    AESIR_TRY(bind(m->ctx));
    TensorRef ref;
    AESIR_TRY(parse_tensor_name(m, name, &ref));
    return model_upload(m, ref, host_data, rows, cols, ggml_type);
}

int32_t aesir_model_get_tensor(aesir_model *m, const char *name, void *host_out, int64_t elements) {
    if (!m || !host_out) return fail(AESIR_ERR_INVALID, "aesir_model_get_tensor: null argument");
    AESIR_TRY(bind(m->ctx));
    TensorRef ref;
    AESIR_TRY(parse_tensor_name(m, name, &ref));
    const TensorPlace p = place_tensor(m, ref);
    if (elements < p.rows * p.cols) return fail(AESIR_ERR_SHAPE, "aesir_model_get_tensor: output too small");
    hipStream_t s = m->ctx->stream;
    if (p.esize == 0) {  // 4-bit types: dequantize on the device (qf_deq16's f16 values)
        void *tmp = nullptr;
        AESIR_HIP_TRY(hipMalloc(&tmp, (size_t)(p.rows * p.cols * 2)));
        int32_t rc = launch_qf_dequant(s, place_qf(p), p.rows, p.cols, p.step, nullptr, tmp, p.cols);
        if (rc == AESIR_OK && hipMemcpyAsync(host_out, tmp, (size_t)(p.rows * p.cols * 2), hipMemcpyDeviceToHost, s) != hipSuccess)
            rc = fail(AESIR_ERR_HIP, "hipMemcpyAsync of the dequantized tensor failed");
        if (hipStreamSynchronize(s) != hipSuccess && rc == AESIR_OK) rc = fail(AESIR_ERR_HIP, "dequantization failed");
        (void)hipFree(tmp);
        return rc;
    }
    if (p.esize == 1) {  // Q8_0: dequantize f16(q * d); the product is exact in f32, so one rounding
        const int64_t nb = p.cols / 32;
        std::vector<int8_t> qs((size_t)(p.rows * p.cols));
        std::vector<uint16_t> ds((size_t)(p.rows * nb));
        AESIR_HIP_TRY(hipMemcpy2DAsync(qs.data(), (size_t)p.cols, p.base, (size_t)p.row_stride, (size_t)p.cols,
                                       (size_t)p.rows, hipMemcpyDeviceToHost, s));
        AESIR_HIP_TRY(hipMemcpy2DAsync(ds.data(), (size_t)nb * 2, p.scale, (size_t)p.scale_stride * 2, (size_t)nb * 2,
                                       (size_t)p.rows, hipMemcpyDeviceToHost, s));
        AESIR_HIP_TRY(hipStreamSynchronize(s));
        uint16_t *o = (uint16_t *)host_out;
        for (int64_t i = 0; i < p.rows * p.cols; i++) o[i] = f32_to_f16_bits((float)qs[i] * f16_bits_to_f32(ds[i / 32]));
        return AESIR_OK;
    }
    AESIR_HIP_TRY(hipMemcpy2DAsync(host_out, (size_t)p.cols * 2, p.base, (size_t)p.row_stride * 2, (size_t)p.cols * 2,
                                   (size_t)p.rows, hipMemcpyDeviceToHost, s));
    AESIR_HIP_TRY(hipStreamSynchronize(s));
    return AESIR_OK;
}

int32_t aesir_model_init_random(aesir_model *m, uint64_t seed, float std, float norm_mean, float norm_std) {
    if (!m) return fail(AESIR_ERR_INVALID, "aesir_model_init_random: null model");
    AESIR_TRY(bind(m->ctx));
    for (const TensorRef &ref : all_tensors(m)) {
        const TensorPlace p = place_tensor(m, ref);
        if (p.esize == 0) {
            AESIR_TRY(launch_qf_fill_random(m->ctx->stream, place_qf(p), p.rows, p.cols, p.step, seed,
                                            (uint64_t)stream_id(ref), std));
            continue;
        }
        if (p.esize == 1) {
            AESIR_TRY(launch_fill_q8_0(m->ctx->stream, p.base, p.row_stride, p.scale, p.scale_stride, p.rows, p.cols,
                                       seed, (uint64_t)stream_id(ref), std));
            continue;
        }
        AESIR_TRY(launch_fill_normal(m->ctx->stream, p.base, p.rows * p.cols, p.cols, p.row_stride, seed,
                                     (uint64_t)stream_id(ref), p.is_norm ? norm_mean : 0.0f,
                                     p.is_norm ? norm_std : std));
    }
    AESIR_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    return AESIR_OK;
}

int32_t aesir_forward_pass(aesir_model *m, const int64_t *tokens, int64_t n_tokens, int64_t start_pos,
                           int64_t *next_token) {
    if (!m || !next_token) return fail(AESIR_ERR_INVALID, "forward_pass: null argument");
    AESIR_TRY(bind(m->ctx));
    if (n_tokens <= 0) {  // inference.mojo:446-447
        *next_token = 0;
        return AESIR_OK;
    }
    if (!tokens) return fail(AESIR_ERR_INVALID, "forward_pass: null token list");
    if (start_pos < 0) return fail(AESIR_ERR_INVALID, "apply_rope: start_pos cannot be negative");
    int64_t idx = start_pos < n_tokens - 1 ? start_pos : n_tokens - 1;  // inference.mojo:449-450
    const int64_t tok = tokens[idx];
    if (tok < 0 || tok >= m->cfg.vocab) return fail(AESIR_ERR_INVALID, "Prompt token ID is outside the embedding vocabulary");
    AESIR_TRY(ensure_rope(m, start_pos + 1));
    return model_step(m, tok, start_pos, next_token);
}

int32_t aesir_forward_pass_no_cache(aesir_model *m, const int64_t *tokens, int64_t n_tokens, int64_t *next_token) {
    if (!m || !next_token) return fail(AESIR_ERR_INVALID, "forward_pass: null argument");
    AESIR_TRY(bind(m->ctx));
    if (n_tokens <= 0) {  // start_pos 0 over an empty list: inference.mojo:446-447
        *next_token = 0;
        return AESIR_OK;
    }
    // inference.mojo:543-546: a new KVCache carved from never-used (zeroed) well memory, then
    // the last token at position len - 1. The rows that attention reads besides the one this
    // step appends are rows [0, min(start_pos, ctx_len)) of every layer: clear them.
    const int64_t start_pos = n_tokens - 1;
    const int64_t rows = start_pos < m->cfg.ctx_len ? start_pos : m->cfg.ctx_len;
    if (rows > 0) {
        const size_t pitch = (size_t)(m->cfg.ctx_len * m->kvd * 2), width = (size_t)(rows * m->kvd * 2);
        AESIR_HIP_TRY(hipMemset2DAsync(m->k_cache, pitch, 0, width, (size_t)m->cfg.n_layers, m->ctx->stream));
        AESIR_HIP_TRY(hipMemset2DAsync(m->v_cache, pitch, 0, width, (size_t)m->cfg.n_layers, m->ctx->stream));
    }
    return aesir_forward_pass(m, tokens, n_tokens, start_pos, next_token);
}

int32_t aesir_model_logits(aesir_model *m, void *host_out) {
    if (!m || !host_out) return fail(AESIR_ERR_INVALID, "aesir_model_logits: null argument");
    return aesir_memcpy_d2h(m->ctx, host_out, m->logits, m->cfg.vocab * 2);
}

int32_t aesir_decode_loop(aesir_model *m, int64_t token, int64_t start_pos, int64_t n_steps, int32_t use_graph,
                          int64_t *out_tokens, float *elapsed_ms) {
    if (!m) return fail(AESIR_ERR_INVALID, "aesir_decode_loop: null model");
    AESIR_TRY(bind(m->ctx));
    if (n_steps <= 0) return fail(AESIR_ERR_INVALID, "aesir_decode_loop: n_steps must be positive");
    if (start_pos < 0) return fail(AESIR_ERR_INVALID, "apply_rope: start_pos cannot be negative");
    if (token < 0 || token >= m->cfg.vocab) return fail(AESIR_ERR_INVALID, "Prompt token ID is outside the embedding vocabulary");
    if (n_steps > m->ring_cap) return fail(AESIR_ERR_INVALID, "aesir_decode_loop: at most %lld steps per call", (long long)m->ring_cap);
    AESIR_TRY(ensure_rope(m, start_pos + n_steps));
    if (use_graph) AESIR_TRY(ensure_graph(m));
    AESIR_TRY(upload_state(m, token, start_pos, 1, m->ring_cap));
    hipStream_t s = m->ctx->stream;
    AESIR_HIP_TRY(hipEventRecord(m->ctx->ev_start, s));
    for (int64_t i = 0; i < n_steps; i++) AESIR_TRY(run_step(m, use_graph != 0));
    AESIR_HIP_TRY(hipEventRecord(m->ctx->ev_stop, s));
    AESIR_HIP_TRY(hipEventSynchronize(m->ctx->ev_stop));
    float ms = 0.0f;
    AESIR_HIP_TRY(hipEventElapsedTime(&ms, m->ctx->ev_start, m->ctx->ev_stop));
    if (elapsed_ms) *elapsed_ms = ms;
    if (out_tokens)
        AESIR_HIP_TRY(hipMemcpy(out_tokens, m->ring, (size_t)n_steps * sizeof(int64_t), hipMemcpyDeviceToHost));
    return AESIR_OK;
}

int32_t aesir_model_fill_kv_random(aesir_model *m, int64_t n_pos, uint64_t seed, float std) {
    if (!m) return fail(AESIR_ERR_INVALID, "aesir_model_fill_kv_random: null model");
    AESIR_TRY(bind(m->ctx));
    if (n_pos <= 0 || n_pos > m->cfg.ctx_len)
        return fail(AESIR_ERR_INVALID, "aesir_model_fill_kv_random: n_pos must be in [1, ctx_len]");
    const int64_t per_layer = m->cfg.ctx_len * m->kvd;
    for (int64_t l = 0; l < m->cfg.n_layers; l++) {
        AESIR_TRY(launch_fill_normal(m->ctx->stream, (uint16_t *)m->k_cache + l * per_layer, n_pos * m->kvd, m->kvd,
                                     m->kvd, seed, 1000000 + 2 * (uint64_t)l, 0.0f, std));
        AESIR_TRY(launch_fill_normal(m->ctx->stream, (uint16_t *)m->v_cache + l * per_layer, n_pos * m->kvd, m->kvd,
                                     m->kvd, seed, 1000001 + 2 * (uint64_t)l, 0.0f, std));
    }
    AESIR_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    return AESIR_OK;
}

int32_t aesir_model_kernel_times(aesir_model *m, int64_t pos, int32_t iters, float *times, int32_t n_times) {
    if (!m || !times || n_times < 7) return fail(AESIR_ERR_INVALID, "aesir_model_kernel_times: need 7 outputs");
    AESIR_TRY(bind(m->ctx));
    if (iters <= 0) return fail(AESIR_ERR_INVALID, "aesir_model_kernel_times: iters must be positive");
    AESIR_TRY(ensure_rope(m, pos + 1));
    AESIR_TRY(upload_state(m, 0, pos, 0, m->ring_cap));
    hipStream_t s = m->ctx->stream;
    const aesir_model_config &c = m->cfg;
    const int64_t d = c.dim;
    // Class k is launched back to back, cycling through the layers so that no layer's weights
    // are re-read from cache; time per launch = HIP-event time / launches.
    for (int cls = 0; cls < 7; cls++) {
        const int64_t per_iter = cls >= 5 ? 1 : c.n_layers;
        auto launch = [&](int64_t l) -> int32_t {
            const ModelLayer &L = m->layers[l];
            switch (cls) {
                case 0: return launch_qkv_rope_kv(s, qkv_args(m, l));
                case 1: return launch_attention_decode(s, attn_args(m, l));
                case 2: return launch_o_residual(m, s, L);
                case 3: return launch_gate_up(m, s, L);
                case 4: return launch_down_residual(m, s, L);
                case 5: return launch_lm_head(s, lm_args(m, false));
                default: return launch_argmax_finish(s, m->lm_parts, lm_head_groups(c.vocab), m->state, nullptr, nullptr);
            }
        };
        int32_t rc = AESIR_OK;
        for (int64_t l = 0; l < per_iter && rc == AESIR_OK; l++) rc = launch(l);  // warm-up
        if (rc != AESIR_OK) return rc;
        AESIR_HIP_TRY(hipEventRecord(m->ctx->ev_start, s));
        for (int32_t it = 0; it < iters && rc == AESIR_OK; it++)
            for (int64_t l = 0; l < per_iter && rc == AESIR_OK; l++) rc = launch(l);
        if (rc != AESIR_OK) return rc;
        AESIR_HIP_TRY(hipEventRecord(m->ctx->ev_stop, s));
        AESIR_HIP_TRY(hipEventSynchronize(m->ctx->ev_stop));
        float ms = 0.0f;
        AESIR_HIP_TRY(hipEventElapsedTime(&ms, m->ctx->ev_start, m->ctx->ev_stop));
        times[cls] = ms / (float)(iters * per_iter);
    }
    return AESIR_OK;
}

int32_t aesir_generation_stop_reason(int64_t token, int64_t eos_token_id, int64_t generated_count,
                                     int64_t max_new_tokens, const int64_t *stop_tokens, int64_t n_stop,
                                     int64_t next_position, int64_t context_length) {
    // aesir.mojo:195-212
    if (eos_token_id >= 0 && token == eos_token_id) return AESIR_STOP_EOS;
    for (int64_t i = 0; i < n_stop; i++)
        if (stop_tokens && stop_tokens[i] == token) return AESIR_STOP_TOKEN;
    if (generated_count >= max_new_tokens) return AESIR_STOP_LENGTH;
    if (next_position >= context_length) return AESIR_STOP_CONTEXT_EXHAUSTED;
    return -1;
}

int32_t aesir_generate(aesir_model *m, const int64_t *prompt, int64_t n_prompt, const aesir_generation_config *gc,
                       int64_t *out_tokens, int64_t *n_out, int32_t *stop_reason) {
    if (!m || !gc || !out_tokens || !n_out || !stop_reason) return fail(AESIR_ERR_INVALID, "aesir_generate: null argument");
    AESIR_TRY(bind(m->ctx));
    *n_out = 0;
    const int64_t ctx_len = m->cfg.ctx_len, max_new = gc->max_new_tokens;
    // GenerationConfig.validate (aesir.mojo:125-128) and _run_generation's prompt checks (:343-346)
    if (max_new <= 0) return fail(AESIR_ERR_INVALID, "GenerationConfig max_new_tokens must be a positive integer");
    if (max_new > ctx_len) return fail(AESIR_ERR_INVALID, "GenerationConfig max_new_tokens exceeds context_length boundary");
    if (n_prompt <= 0 || !prompt) return fail(AESIR_ERR_INVALID, "RuneWeaver produced no prompt tokens");
    if (n_prompt > ctx_len) return fail(AESIR_ERR_INVALID, "Prompt token count exceeds the model context length");
    std::vector<int64_t> cur(prompt, prompt + n_prompt);
    int64_t next = 0;
    if (gc->batched_prefill)
        AESIR_TRY(model_prefill(m, cur.data(), n_prompt, 0, &next));
    else
        for (int64_t p = 0; p < n_prompt; p++) AESIR_TRY(aesir_forward_pass(m, cur.data(), (int64_t)cur.size(), p, &next));
    int32_t reason = -1;
    const int64_t eos = m->cfg.eos_token_id;
    for (int64_t it = 0; it < max_new; it++) {  // aesir.mojo:381-445
        out_tokens[(*n_out)++] = next;
        cur.push_back(next);
        if (next == eos) {
            reason = AESIR_STOP_EOS;
            break;
        }
        bool is_stop = false;
        for (int64_t s = 0; s < gc->n_stop_tokens; s++) is_stop |= gc->stop_tokens[s] == next;
        if (is_stop) {
            reason = AESIR_STOP_TOKEN;
            break;
        }
        const int64_t next_position = (int64_t)cur.size() - 1;
        reason = aesir_generation_stop_reason(next, eos, *n_out, max_new, gc->stop_tokens, gc->n_stop_tokens,
                                              next_position, ctx_len);
        if (reason >= 0) break;
        AESIR_TRY(aesir_forward_pass(m, cur.data(), (int64_t)cur.size(), next_position, &next));
    }
    if (reason < 0) reason = AESIR_STOP_LENGTH;
    *stop_reason = reason;
    return AESIR_OK;
}

}  // extern "C"
