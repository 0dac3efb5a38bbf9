// GGUF v3 loader: file -> validated Llama F16 contract -> model in the HBM arena.
//
// Restates GGUFSeer (loader/gguf.mojo:183-690): bounds-checked parsing of the header, metadata
// and tensor table of a read-only mmap, the same accepted keys and types, the same errors
// (message text included), then _validate_required_tensors. Where the reference aliases F16
// tensors into the mmap, this loader uploads them once into the model's arena (Q/K/V
// concatenated, gate/up interleaved); F32 norms are rounded to f16 as the reference does.
// One extension: each matrix may also have a block type, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q2_K,
// Q3_K, Q4_K, Q5_K or Q6_K (GGML types 8, 2, 3, 6, 7, 10, 11, 12, 13, 14), matrix by matrix (files
// such as Q4_K_M mix them); the model keeps each matrix in its own type or in f16 (the reference
// loader stops at "Real inference slice supports only F16 and F32 tensors"). Any other matrix
// type is refused with "GGUF required tensor has an invalid type".
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <set>
#include <string>

#include "common.hpp"
#include "model.hpp"

namespace aesir {
namespace {

struct GgufTensor {
    std::string name;
    int64_t rows, cols;
    uint32_t type;
    int64_t offset;  // absolute file offset
};

struct Gguf {
    const uint8_t *p = nullptr;
    int64_t size = 0;
    int fd = -1;
    // metadata (GGUFModelConfig, loader/gguf.mojo:83-149)
    std::string arch;
    int64_t context_length = 0, embedding_length = 0, feed_forward_length = 0, block_count = 0;
    int64_t head_count = 0, head_count_kv = 0, rope_dimension_count = 0;
    float rms_epsilon = 1e-5f;
    float rope_freq_base = 10000.0f;
    bool has_freq_base = false;
    int64_t unknown_token_id = 0, bos_token_id = 1, eos_token_id = 2;
    int64_t n_tokens = 0, n_scores = 0, n_types = 0;
    int64_t alignment = 32;
    int64_t tensor_count = 0, kv_count = 0;
    std::vector<GgufTensor> tensors;
    std::map<std::string, size_t> by_name;

    ~Gguf() {
        if (p) munmap((void *)p, (size_t)size);
        if (fd >= 0) close(fd);
    }

    // _require_range (loader/gguf.mojo:218-222)
    int32_t need(int64_t off, int64_t n) const {
        if (off < 0 || n < 0) return fail(AESIR_ERR_FORMAT, "GGUF contains a negative byte range");
        if (off > size || n > size - off) return fail(AESIR_ERR_FORMAT, "GGUF is truncated or contains an out-of-range offset");
        return AESIR_OK;
    }
    template <class T>
    int32_t rd(int64_t off, T *out) const {
        AESIR_TRY(need(off, (int64_t)sizeof(T)));
        std::memcpy(out, p + off, sizeof(T));
        return AESIR_OK;
    }
    int32_t rd_string(int64_t off, std::string *s, int64_t *end) const {
        uint64_t n;
        AESIR_TRY(rd(off, &n));
        if (n > (uint64_t)size) return fail(AESIR_ERR_FORMAT, "GGUF is truncated or contains an out-of-range offset");
        AESIR_TRY(need(off + 8, (int64_t)n));
        if (s) s->assign((const char *)p + off + 8, (size_t)n);
        *end = off + 8 + (int64_t)n;
        return AESIR_OK;
    }
    // skip_value (loader/gguf.mojo:247-273)
    int32_t skip(uint32_t t, int64_t off, int64_t *end) const {
        if (t == 0 || t == 1 || t == 7) return need(off, 1) ? AESIR_ERR_FORMAT : (*end = off + 1, AESIR_OK);
        if (t == 2 || t == 3) return need(off, 2) ? AESIR_ERR_FORMAT : (*end = off + 2, AESIR_OK);
        if (t == 4 || t == 5 || t == 6) return need(off, 4) ? AESIR_ERR_FORMAT : (*end = off + 4, AESIR_OK);
        if (t == 10 || t == 11 || t == 12) return need(off, 8) ? AESIR_ERR_FORMAT : (*end = off + 8, AESIR_OK);
        if (t == 8) return rd_string(off, nullptr, end);
        if (t == 9) {
            uint32_t at;
            uint64_t n;
            AESIR_TRY(rd(off, &at));
            AESIR_TRY(rd(off + 4, &n));
            if (at >= 13) return fail(AESIR_ERR_FORMAT, "GGUF array contains an invalid element type");
            if (n > (uint64_t)size) return fail(AESIR_ERR_FORMAT, "GGUF array length exceeds the file size");
            int64_t cur = off + 12;
            static const int fixed[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
            if (at != 8 && at != 9) {
                AESIR_TRY(need(cur, (int64_t)n * fixed[at]));
                *end = cur + (int64_t)n * fixed[at];
                return AESIR_OK;
            }
            for (uint64_t i = 0; i < n; i++) AESIR_TRY(skip(at, cur, &cur));
            *end = cur;
            return AESIR_OK;
        }
        return fail(AESIR_ERR_FORMAT, "GGUF contains an invalid metadata value type");
    }
    int32_t array_len(int64_t off, uint32_t want_type, const char *msg, int64_t *n_out, int64_t *end) const {
        uint32_t at;
        uint64_t n;
        AESIR_TRY(rd(off, &at));
        AESIR_TRY(rd(off + 4, &n));
        if (at != want_type) return fail(AESIR_ERR_FORMAT, "%s", msg);
        *n_out = (int64_t)n;
        return skip(9, off, end);
    }
};

int32_t u32_at(const Gguf &g, int64_t off, int64_t *out) {
    uint32_t v;
    AESIR_TRY(g.rd(off, &v));
    *out = v;
    return AESIR_OK;
}

// _parse_metadata_value (loader/gguf.mojo:322-377): only the listed keys with the listed types
// are read; everything else is skipped.
int32_t parse_kv(Gguf &g, const std::string &key, uint32_t t, int64_t off, int64_t *end) {
    if (key == "tokenizer.ggml.tokens") {
        if (t != 9) return fail(AESIR_ERR_FORMAT, "tokenizer.ggml.tokens is not an array");
        return g.array_len(off, 8, "tokenizer.ggml.tokens must be a string array", &g.n_tokens, end);
    }
    if (key == "tokenizer.ggml.scores") {
        if (t != 9) return fail(AESIR_ERR_FORMAT, "tokenizer.ggml.scores is not an array");
        return g.array_len(off, 6, "tokenizer.ggml.scores must be a float32 array", &g.n_scores, end);
    }
    if (key == "tokenizer.ggml.token_type") {
        if (t != 9) return fail(AESIR_ERR_FORMAT, "tokenizer.ggml.token_type is not an array");
        return g.array_len(off, 5, "tokenizer.ggml.token_type must be an int32 array", &g.n_types, end);
    }
    if (key == "general.architecture" && t == 8) {
        int64_t e;
        AESIR_TRY(g.rd_string(off, &g.arch, &e));
    } else if (t == 4) {
        int64_t v;
        AESIR_TRY(u32_at(g, off, &v));
        if (key == "llama.context_length") g.context_length = v;
        else if (key == "llama.embedding_length") g.embedding_length = v;
        else if (key == "llama.feed_forward_length") g.feed_forward_length = v;
        else if (key == "llama.block_count") g.block_count = v;
        else if (key == "llama.attention.head_count") g.head_count = v;
        else if (key == "llama.attention.head_count_kv") g.head_count_kv = v;
        else if (key == "llama.rope.dimension_count") g.rope_dimension_count = v;
        else if (key == "general.alignment") g.alignment = v;
        else if (key == "tokenizer.ggml.unknown_token_id") g.unknown_token_id = v;
        else if (key == "tokenizer.ggml.bos_token_id") g.bos_token_id = v;
        else if (key == "tokenizer.ggml.eos_token_id") g.eos_token_id = v;
    } else if (t == 6) {
        float v;
        AESIR_TRY(g.rd(off, &v));
        if (key == "llama.attention.layer_norm_rms_epsilon") g.rms_epsilon = v;
        // Recorded but, like the reference (inference.mojo:200), not applied: theta stays 10000.
        if (key == "llama.rope.freq_base") {
            g.rope_freq_base = v;
            g.has_freq_base = true;
        }
    }
    return g.skip(t, off, end);
}

int32_t parse(Gguf &g, const char *path) {
    g.fd = open(path, O_RDONLY);
    if (g.fd < 0) return fail(AESIR_ERR_IO, "Failed to open GGUF model: %s", path);
    struct stat st;
    if (fstat(g.fd, &st) != 0) return fail(AESIR_ERR_IO, "Failed to open GGUF model: %s", path);
    g.size = (int64_t)st.st_size;
    if (g.size < 24) return fail(AESIR_ERR_FORMAT, "GGUF file is smaller than the v3 header");
    void *mp = mmap(nullptr, (size_t)g.size, PROT_READ, MAP_PRIVATE, g.fd, 0);
    if (mp == MAP_FAILED) return fail(AESIR_ERR_IO, "Failed to mmap GGUF model");
    g.p = (const uint8_t *)mp;
    // _parse_header (loader/gguf.mojo:405-416)
    uint32_t magic, version;
    uint64_t tc, kc;
    AESIR_TRY(g.rd(0, &magic));
    if (magic != 0x46554747u) return fail(AESIR_ERR_FORMAT, "GGUF magic bytes are invalid");
    AESIR_TRY(g.rd(4, &version));
    if (version != 3) return fail(AESIR_ERR_FORMAT, "Only GGUF version 3 is supported by this inference slice");
    AESIR_TRY(g.rd(8, &tc));
    AESIR_TRY(g.rd(16, &kc));
    if (tc > (uint64_t)g.size || kc > (uint64_t)g.size) return fail(AESIR_ERR_FORMAT, "GGUF entry counts exceed the file size");
    g.tensor_count = (int64_t)tc;
    g.kv_count = (int64_t)kc;
    // _parse_metadata (loader/gguf.mojo:418-448)
    int64_t cur = 24;
    std::set<std::string> seen;
    for (int64_t i = 0; i < g.kv_count; i++) {
        std::string key;
        AESIR_TRY(g.rd_string(cur, &key, &cur));
        if (!seen.insert(key).second) return fail(AESIR_ERR_FORMAT, "GGUF contains duplicate metadata key: %s", key.c_str());
        uint32_t t;
        AESIR_TRY(g.rd(cur, &t));
        cur += 4;
        AESIR_TRY(parse_kv(g, key, t, cur, &cur));
    }
    if (g.alignment <= 0 || g.alignment > 4096 || (g.alignment & (g.alignment - 1)) != 0)
        return fail(AESIR_ERR_FORMAT, "GGUF alignment must be a power of two up to 4096");
    // GGUFModelConfig.validate (loader/gguf.mojo:133-149)
    if (g.arch != "llama") return fail(AESIR_ERR_FORMAT, "GGUF architecture is not supported: %s", g.arch.c_str());
    if (g.context_length <= 0 || g.embedding_length <= 0) return fail(AESIR_ERR_FORMAT, "GGUF model dimensions are incomplete");
    if (g.feed_forward_length <= 0 || g.block_count <= 0) return fail(AESIR_ERR_FORMAT, "GGUF layer metadata is incomplete");
    if (g.head_count <= 0 || g.head_count_kv <= 0) return fail(AESIR_ERR_FORMAT, "GGUF attention metadata is incomplete");
    if (g.embedding_length % g.head_count != 0) return fail(AESIR_ERR_FORMAT, "GGUF embedding length is not divisible by head count");
    if (g.head_count % g.head_count_kv != 0) return fail(AESIR_ERR_FORMAT, "GGUF query heads are not divisible by KV heads");
    if (g.rope_dimension_count != g.embedding_length / g.head_count)
        return fail(AESIR_ERR_FORMAT, "GGUF RoPE dimension does not match attention head size");
    // RuneWeaver.validate_vocabulary (loader/tokenizer.mojo:69-84)
    if (g.n_tokens <= 0) return fail(AESIR_ERR_FORMAT, "Tokenizer vocabulary is empty");
    if (g.n_scores != g.n_tokens) return fail(AESIR_ERR_FORMAT, "Tokenizer scores length does not match vocab_size");
    if (g.n_types != g.n_tokens) return fail(AESIR_ERR_FORMAT, "Tokenizer token_types length does not match vocab_size");
    if (g.unknown_token_id < 0 || g.unknown_token_id >= g.n_tokens) return fail(AESIR_ERR_FORMAT, "Tokenizer unknown_token_id is out of bounds");
    if (g.bos_token_id < 0 || g.bos_token_id >= g.n_tokens) return fail(AESIR_ERR_FORMAT, "Tokenizer bos_token_id is out of bounds");
    if (g.eos_token_id < 0 || g.eos_token_id >= g.n_tokens) return fail(AESIR_ERR_FORMAT, "Tokenizer eos_token_id is out of bounds");
    // _parse_tensors (loader/gguf.mojo:501-550)
    std::vector<GgufTensor> raw;
    for (int64_t i = 0; i < g.tensor_count; i++) {
        GgufTensor t;
        AESIR_TRY(g.rd_string(cur, &t.name, &cur));
        uint32_t nd;
        AESIR_TRY(g.rd(cur, &nd));
        cur += 4;
        if (nd == 0 || nd > 2) return fail(AESIR_ERR_FORMAT, "Inference tensor must have one or two dimensions: %s", t.name.c_str());
        uint64_t ne0, ne1 = 1;
        AESIR_TRY(g.rd(cur, &ne0));
        cur += 8;
        if (nd == 2) {
            AESIR_TRY(g.rd(cur, &ne1));
            cur += 8;
        }
        if ((int64_t)ne0 <= 0 || (int64_t)ne1 <= 0) return fail(AESIR_ERR_FORMAT, "GGUF tensor has a non-positive dimension: %s", t.name.c_str());
        t.cols = (int64_t)ne0;
        t.rows = (int64_t)ne1;
        AESIR_TRY(g.rd(cur, &t.type));
        cur += 4;
        uint64_t off;
        AESIR_TRY(g.rd(cur, &off));
        cur += 8;
        t.offset = (int64_t)off;
        raw.push_back(t);
    }
    const int64_t data_offset = (cur + g.alignment - 1) / g.alignment * g.alignment;
    AESIR_TRY(g.need(data_offset, 0));
    for (auto &t : raw) {  // _map_tensor (loader/gguf.mojo:465-499)
        if (g.by_name.count(t.name)) return fail(AESIR_ERR_FORMAT, "GGUF contains a duplicate tensor name: %s", t.name.c_str());
        // F16 and F32 as the reference loader; the block types beyond it (Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q2_K,
        // Q3_K, Q4_K, Q5_K, Q6_K) by their GGML block geometry. Every size product is overflow-checked before
        // any range check.
        const int64_t bytes = ggml_tensor_bytes(t.type, t.rows, t.cols);
        if (bytes == -1) return fail(AESIR_ERR_FORMAT, "Real inference slice supports only F16 and F32 tensors");
        if (bytes == -2)
            return fail(AESIR_ERR_FORMAT, "GGUF tensor row length is not a multiple of its block size: %s", t.name.c_str());
        if (bytes < 0 || bytes > g.size)
            return fail(AESIR_ERR_FORMAT, "GGUF tensor byte size overflows the file: %s", t.name.c_str());
        if (t.offset < 0 || t.offset % g.alignment != 0)
            return fail(AESIR_ERR_FORMAT, "GGUF tensor offset is not correctly aligned: %s", t.name.c_str());
        if (t.offset > g.size) return fail(AESIR_ERR_FORMAT, "GGUF is truncated or contains an out-of-range offset");
        t.offset += data_offset;
        AESIR_TRY(g.need(t.offset, bytes));
        g.by_name[t.name] = g.tensors.size();
        g.tensors.push_back(t);
    }
    return AESIR_OK;
}

}  // namespace
}  // namespace aesir

using namespace aesir;

namespace aesir {
namespace {

std::vector<std::string> required_tensors(const Gguf &g) {
    std::vector<std::string> required = {"token_embd.weight", "output_norm.weight", "output.weight"};
    static const char *per[] = {"attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                                "ffn_norm", "ffn_gate", "ffn_up", "ffn_down"};
    for (int64_t l = 0; l < g.block_count; l++)
        for (const char *b : per) required.push_back("blk." + std::to_string(l) + "." + b + ".weight");
    return required;
}

// Types a matrix may have: F16 as the reference requires, and the block types this library adds
// (Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K), each matrix its own (GGUF files
// mix them: Q4_K_M and the like).
bool matrix_type_ok(uint32_t t) { return t == AESIR_GGML_F16 || gguf_block_elems((int32_t)t) != 0; }

// Expected (rows, cols) of a required tensor (loader/gguf.mojo:597-628); *norm for the F32 norms.
void expected_shape(const Gguf &g, const std::string &name, int64_t vocab, int64_t *rows, int64_t *cols, bool *norm) {
    const int64_t d = g.embedding_length, kvd = d / g.head_count * g.head_count_kv, f = g.feed_forward_length;
    auto ends = [&](const char *suf) {
        const size_t n = std::strlen(suf);
        return name.size() >= n && name.compare(name.size() - n, n, suf) == 0;
    };
    *norm = false;
    if (name == "token_embd.weight" || name == "output.weight") { *rows = vocab; *cols = d; }
    else if (ends("norm.weight")) { *rows = 1; *cols = d; *norm = true; }
    else if (ends("attn_q.weight") || ends("attn_output.weight")) { *rows = d; *cols = d; }
    else if (ends("attn_k.weight") || ends("attn_v.weight")) { *rows = kvd; *cols = d; }
    else if (ends("ffn_gate.weight") || ends("ffn_up.weight")) { *rows = f; *cols = d; }
    else { *rows = d; *cols = f; }  // ffn_down
}

// _validate_required_tensors (loader/gguf.mojo:567-628): presence first, then shapes/types.
int32_t validate_required(const Gguf &g) {
    const std::vector<std::string> required = required_tensors(g);
    for (auto &r : required)
        if (!g.by_name.count(r)) return fail(AESIR_ERR_FORMAT, "GGUF is missing required tensor: %s", r.c_str());
    const int64_t vocab = g.tensors[g.by_name.at("token_embd.weight")].rows;
    for (auto &r : required) {
        const GgufTensor &t = g.tensors[g.by_name.at(r)];
        int64_t rows, cols;
        bool norm;
        expected_shape(g, r, vocab, &rows, &cols, &norm);
        if (t.rows != rows || t.cols != cols) return fail(AESIR_ERR_FORMAT, "GGUF required tensor has an invalid shape: %s", r.c_str());
        if (norm ? t.type != AESIR_GGML_F32 : !matrix_type_ok(t.type))
            return fail(AESIR_ERR_FORMAT, "GGUF required tensor has an invalid type: %s", r.c_str());
    }
    return AESIR_OK;
}

// The matrices' types in aesir_model_create_mixed's order.
WeightTypes weight_types(const Gguf &g) {
    auto type = [&](const std::string &n) { return (int32_t)g.tensors[g.by_name.at(n)].type; };
    WeightTypes t;
    t.embd = type("token_embd.weight");
    t.out = type("output.weight");
    for (int64_t l = 0; l < g.block_count; l++) {
        const std::string b = "blk." + std::to_string(l) + ".";
        t.layers.push_back(LayerTypes{type(b + "attn_q.weight"), type(b + "attn_k.weight"), type(b + "attn_v.weight"),
                                      type(b + "attn_output.weight"), type(b + "ffn_gate.weight"),
                                      type(b + "ffn_up.weight"), type(b + "ffn_down.weight")});
    }
    return t;
}

void fill_config(const Gguf &g, int64_t ctx_len_override, aesir_model_config *c) {
    *c = aesir_model_config{};
    c->dim = g.embedding_length;
    c->n_layers = g.block_count;
    c->n_heads = g.head_count;
    c->n_kv_heads = g.head_count_kv;
    c->ffn = g.feed_forward_length;
    c->vocab = g.tensors[g.by_name.at("token_embd.weight")].rows;
    c->ctx_len = ctx_len_override > 0 ? ctx_len_override : g.context_length;
    c->rms_eps = g.rms_epsilon;
    c->rope_theta = 10000.0f;  // the reference never reads llama.rope.freq_base (inference.mojo:200)
    c->bos_token_id = g.bos_token_id;
    c->eos_token_id = g.eos_token_id;
}

}  // namespace
}  // namespace aesir

extern "C" int32_t aesir_gguf_inspect(const char *path, aesir_model_config *cfg, float *rope_freq_base) {
    clear_error();
    if (!path || !cfg) return fail(AESIR_ERR_INVALID, "aesir_gguf_inspect: null argument");
    Gguf g;
    AESIR_TRY(parse(g, path));
    AESIR_TRY(validate_required(g));
    fill_config(g, 0, cfg);
    if (rope_freq_base) *rope_freq_base = g.has_freq_base ? g.rope_freq_base : 10000.0f;
    return AESIR_OK;
}

extern "C" int32_t aesir_model_load_gguf(aesir_ctx *ctx, const char *path, int64_t ctx_len_override, aesir_model **out) {
    AESIR_TRY(bind(ctx));
    if (!path || !out) return fail(AESIR_ERR_INVALID, "aesir_model_load_gguf: null argument");
    *out = nullptr;
    Gguf g;
    AESIR_TRY(parse(g, path));
    AESIR_TRY(validate_required(g));
    const std::vector<std::string> required = required_tensors(g);
    aesir_model_config c{};
    fill_config(g, ctx_len_override, &c);
    aesir_model *m = nullptr;
    AESIR_TRY(model_create(ctx, &c, weight_types(g), &m));
    for (auto &r : required) {
        const GgufTensor &t = g.tensors[g.by_name.at(r)];
        TensorRef ref;
        int32_t rc = parse_tensor_name(m, r.c_str(), &ref);
        if (rc == AESIR_OK) rc = model_upload(m, ref, g.p + t.offset, t.rows, t.cols, (int32_t)t.type);
        if (rc != AESIR_OK) {
            std::string msg = aesir_last_error();
            ctx->well_offset = m->well_start;
            aesir_model_destroy(m);
            return fail(rc, "%s", msg.c_str());
        }
    }
    *out = m;
    return AESIR_OK;
}
