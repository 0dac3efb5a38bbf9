// Internal host-side definitions shared by the translation units of libaesir_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "aesir_hip.h"

namespace aesir {

// ------------------------------------------------------------------ errors

// Records the message for aesir_last_error() and returns `code`.
int32_t fail(int32_t code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

#define AESIR_HIP_TRY(expr)                                                                        \
    do {                                                                                           \
        hipError_t _e = (expr);                                                                    \
        if (_e != hipSuccess)                                                                      \
            return ::aesir::fail(AESIR_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(_e));  \
    } while (0)

#define AESIR_TRY(expr)                                                                            \
    do {                                                                                           \
        int32_t _rc = (expr);                                                                      \
        if (_rc != AESIR_OK) return _rc;                                                           \
    } while (0)

// Checks the launch that was just enqueued.
#define AESIR_LAUNCH_CHECK(name)                                                                   \
    do {                                                                                           \
        hipError_t _e = hipGetLastError();                                                         \
        if (_e != hipSuccess)                                                                      \
            return ::aesir::fail(AESIR_ERR_HIP, "launch of %s failed: %s", name, hipGetErrorString(_e)); \
    } while (0)

// Raises a kernel's dynamic LDS limit to `bytes` (above the 64 KB default) once per device: HIP
// keeps the attribute per function and device. `done` is the caller's static bitmask for that
// kernel (bit d = device ordinal d < 64; higher ordinals set the attribute on every call).
inline int32_t raise_lds_limit(const void *fn, int bytes, std::atomic<uint64_t> &done) {
    int dev = 0;
    AESIR_HIP_TRY(hipGetDevice(&dev));
    const uint64_t bit = dev < 64 ? (uint64_t)1 << dev : 0;
    if (bit && (done.load(std::memory_order_relaxed) & bit)) return AESIR_OK;
    AESIR_HIP_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    done.fetch_or(bit, std::memory_order_relaxed);
    return AESIR_OK;
}

// ------------------------------------------------------------------ checked sizes

// a * b, or -1 when an operand is negative or the product overflows int64 (sizes derived from
// file metadata must never wrap).
inline int64_t mul_checked(int64_t a, int64_t b) {
    int64_t r;
    if (a < 0 || b < 0 || __builtin_mul_overflow(a, b, &r)) return -1;
    return r;
}
inline int64_t mul_checked(int64_t a, int64_t b, int64_t c) { return a < 0 || b < 0 ? -1 : mul_checked(mul_checked(a, b), c); }
inline int64_t mul_checked(int64_t a, int64_t b, int64_t c, int64_t d) {
    return mul_checked(mul_checked(a, b, c), d);
}

// GGML block geometry: elements per block and bytes per block of a tensor type (0 if the type
// is not one this library stores).
struct GgmlBlock {
    int64_t elems, bytes;
};
inline GgmlBlock ggml_block(int64_t type) {
    switch (type) {
        case AESIR_GGML_F32: return {1, 4};
        case AESIR_GGML_F16: return {1, 2};
        case AESIR_GGML_Q8_0: return {32, 34};
        case AESIR_GGML_Q4_0: return {32, 18};
        case AESIR_GGML_Q4_1: return {32, 20};
        case AESIR_GGML_Q5_0: return {32, 22};
        case AESIR_GGML_Q5_1: return {32, 24};
        case AESIR_GGML_Q2_K: return {256, 84};
        case AESIR_GGML_Q3_K: return {256, 110};
        case AESIR_GGML_Q4_K: return {256, 144};
        case AESIR_GGML_Q5_K: return {256, 176};
        case AESIR_GGML_Q6_K: return {256, 210};
        default: return {0, 0};
    }
}
inline const char *ggml_type_name(int64_t type) {
    switch (type) {
        case AESIR_GGML_F32: return "F32";
        case AESIR_GGML_F16: return "F16";
        case AESIR_GGML_Q4_0: return "Q4_0";
        case AESIR_GGML_Q4_1: return "Q4_1";
        case AESIR_GGML_Q5_0: return "Q5_0";
        case AESIR_GGML_Q5_1: return "Q5_1";
        case AESIR_GGML_Q8_0: return "Q8_0";
        case AESIR_GGML_Q2_K: return "Q2_K";
        case AESIR_GGML_Q3_K: return "Q3_K";
        case AESIR_GGML_Q4_K: return "Q4_K";
        case AESIR_GGML_Q5_K: return "Q5_K";
        case AESIR_GGML_Q6_K: return "Q6_K";
        default: return "?";
    }
}
// Bytes of a rows x cols tensor of a GGML type: -1 for an unknown type, -2 when cols is not a
// multiple of the block, -3 on overflow.
inline int64_t ggml_tensor_bytes(int64_t type, int64_t rows, int64_t cols) {
    const GgmlBlock b = ggml_block(type);
    if (b.elems == 0) return -1;
    if (cols % b.elems != 0) return -2;
    const int64_t r = mul_checked(rows, cols / b.elems, b.bytes);
    return r < 0 ? -3 : r;
}

// ------------------------------------------------------------------ f16 on the host

uint16_t f32_to_f16_bits(float f);  // round to nearest even
float f16_bits_to_f32(uint16_t h);

// ------------------------------------------------------------------ context

// Cached cos/sin table for one (theta, head_dim): [n_pos][head_dim/2] pairs of f16 (cos, sin),
// built on the host with the reference's f32 expressions (compute.mojo:2227-2230).
struct RopeTable {
    float theta = 0.0f;
    int64_t head_dim = 0;
    int64_t n_pos = 0;
    void *dev = nullptr;
};

struct SamplerWork;  // device workspace of aesir_sample_token (sampler.hip)

// Device scratch owned by the context for the standalone kernel entry points.
struct CtxScratch {
    void *base = nullptr;
    int64_t bytes = 0;
    // carved regions
    float *attn_part = nullptr;     // attention partials (m, l, acc)
    int64_t attn_part_floats = 0;
    void *argmax_part = nullptr;    // argmax partials
    int64_t argmax_part_entries = 0;
    int64_t *result = nullptr;      // device int64 results
};

}  // namespace aesir

struct aesir_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    char *well_base = nullptr;
    int64_t well_capacity = 0;  // f16 elements
    int64_t well_offset = 0;    // f16 elements
    int cu_count = 0;
    int64_t hbm_bytes = 0;
    char arch[64] = {0};
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;
    bool timer_running = false;
    int64_t live_models = 0;  // models created on this context and not yet destroyed
    aesir::CtxScratch scratch;
    std::vector<aesir::RopeTable> rope_tables;
    int64_t *pinned_i64 = nullptr;  // small pinned staging area (64 entries)
    aesir::SamplerWork *sampler = nullptr;  // grown on the first aesir_sample_token call
    void *blas = nullptr;  // hipBLASLt handle and per-shape plans, made by the first library GEMM
};

struct aesir_kv {
    aesir_ctx *ctx = nullptr;
    uint16_t *k = nullptr;  // [num_layers * max_seq][hidden_dim]
    uint16_t *v = nullptr;
    int64_t max_seq = 0, hidden_dim = 0, num_layers = 0;
};

namespace aesir {

// Makes ctx->device current for the calling thread.
int32_t bind(aesir_ctx *ctx);
// Returns (building if needed) a RoPE table covering positions [0, min_pos).
int32_t rope_table(aesir_ctx *ctx, float theta, int64_t head_dim, int64_t min_pos, const void **table);
// Frees the sampler workspace of a context.
void sampler_release(aesir_ctx *ctx);
// Frees a context's hipBLASLt state (blas.hip).
void blas_release(aesir_ctx *ctx);
// Bump allocation in bytes from the well (256-byte aligned).
int32_t well_alloc_bytes(aesir_ctx *ctx, int64_t bytes, void **out);

}  // namespace aesir
