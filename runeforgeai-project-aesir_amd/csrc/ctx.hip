// Context, HBM arena (MimirWell), copies, timers and errors of libaesir_hip.so.
#include <cmath>
#include <cstring>
#include <mutex>

#include "common.hpp"

namespace aesir {

static thread_local char g_err[1024];

int32_t fail(int32_t code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_err[0] = 0; }

uint16_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;  // round to nearest even
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

float f16_bits_to_f32(uint16_t b) {
    _Float16 h;
    std::memcpy(&h, &b, 2);
    return (float)h;
}

int32_t bind(aesir_ctx *ctx) {
    if (!ctx) return fail(AESIR_ERR_INVALID, "aesir: null context");
    AESIR_HIP_TRY(hipSetDevice(ctx->device));
    return AESIR_OK;
}

int32_t well_alloc_bytes(aesir_ctx *ctx, int64_t bytes, void **out) {
    if (bytes <= 0) return fail(AESIR_ERR_INVALID, "MimirWell: allocation count must be positive");
    // 256-byte alignment in f16 elements keeps every 16-byte vector load aligned.
    int64_t start = (ctx->well_offset + 127) & ~int64_t(127);
    int64_t elems = (bytes + 1) / 2;
    if (start + elems > ctx->well_capacity) return fail(AESIR_ERR_EXHAUSTED, "MimirWell: memory pool exhausted");
    *out = ctx->well_base + start * 2;
    ctx->well_offset = start + elems;
    return AESIR_OK;
}

// Host computation follows apply_rope's per-pair angle exactly (compute.mojo:2227-2230):
// freq = 1 / theta^(i/hd) in f32, val = f32(pos) * freq, cos/sin in f32, rounded to f16.
int32_t rope_table(aesir_ctx *ctx, float theta, int64_t head_dim, int64_t min_pos, const void **table) {
    for (auto &t : ctx->rope_tables) {
        if (t.theta == theta && t.head_dim == head_dim && t.n_pos >= min_pos) {
            *table = t.dev;
            return AESIR_OK;
        }
    }
    int64_t n_pos = 1;
    while (n_pos < min_pos) n_pos <<= 1;
    if (n_pos < 4096) n_pos = 4096;
    const int64_t half = head_dim / 2;
    std::vector<uint16_t> host((size_t)(n_pos * half * 2));
    std::vector<float> freq((size_t)half);
    for (int64_t j = 0; j < half; j++)
        freq[j] = 1.0f / powf(theta, (float)(2 * j) / (float)head_dim);
    for (int64_t p = 0; p < n_pos; p++) {
        for (int64_t j = 0; j < half; j++) {
            float val = (float)p * freq[j];
            host[(p * half + j) * 2 + 0] = f32_to_f16_bits(cosf(val));
            host[(p * half + j) * 2 + 1] = f32_to_f16_bits(sinf(val));
        }
    }
    // Replace a smaller table for the same (theta, head_dim).
    for (auto it = ctx->rope_tables.begin(); it != ctx->rope_tables.end(); ++it) {
        if (it->theta == theta && it->head_dim == head_dim) {
            AESIR_HIP_TRY(hipStreamSynchronize(ctx->stream));
            AESIR_HIP_TRY(hipFree(it->dev));
            ctx->rope_tables.erase(it);
            break;
        }
    }
    RopeTable t;
    t.theta = theta;
    t.head_dim = head_dim;
    t.n_pos = n_pos;
    AESIR_HIP_TRY(hipMalloc(&t.dev, host.size() * 2));
    AESIR_HIP_TRY(hipMemcpy(t.dev, host.data(), host.size() * 2, hipMemcpyHostToDevice));
    ctx->rope_tables.push_back(t);
    *table = t.dev;
    return AESIR_OK;
}

}  // namespace aesir

using namespace aesir;

extern "C" {

const char *aesir_last_error(void) { return g_err; }

int32_t aesir_abi_version(void) { return AESIR_ABI_VERSION; }

int32_t aesir_ctx_create(int32_t device, int64_t well_bytes, aesir_ctx **out) {
    clear_error();
    if (!out) return fail(AESIR_ERR_INVALID, "aesir_ctx_create: null output handle");
    *out = nullptr;
    if (well_bytes <= 0) return fail(AESIR_ERR_INVALID, "MimirWell: pool size must be positive");
    int n = 0;
    AESIR_HIP_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n)
        return fail(AESIR_ERR_INVALID, "aesir_ctx_create: device %d not present (%d visible)", device, n);
    AESIR_HIP_TRY(hipSetDevice(device));
    hipDeviceProp_t prop;
    AESIR_HIP_TRY(hipGetDeviceProperties(&prop, device));
    auto *ctx = new aesir_ctx();
    ctx->device = device;
    ctx->cu_count = prop.multiProcessorCount;
    ctx->hbm_bytes = (int64_t)prop.totalGlobalMem;
    std::snprintf(ctx->arch, sizeof ctx->arch, "%s", prop.gcnArchName);
    auto cleanup = [&](int32_t rc) {
        aesir_ctx_destroy(ctx);
        return rc;
    };
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess)
        return cleanup(fail(AESIR_ERR_HIP, "hipStreamCreate failed"));
    ctx->well_capacity = well_bytes / 2;
    if (hipMalloc((void **)&ctx->well_base, (size_t)ctx->well_capacity * 2) != hipSuccess)
        return cleanup(fail(AESIR_ERR_EXHAUSTED, "MimirWell: cannot reserve %lld bytes of HBM", (long long)well_bytes));
    // MimirWell zeroes its pool at creation (core/mimir_well.mojo:541).
    if (hipMemsetAsync(ctx->well_base, 0, (size_t)ctx->well_capacity * 2, ctx->stream) != hipSuccess)
        return cleanup(fail(AESIR_ERR_HIP, "hipMemsetAsync of the well failed"));
    // Context scratch for the standalone kernels: attention partials (4M floats), 64K argmax
    // partials, 64 result slots.
    CtxScratch &s = ctx->scratch;
    s.attn_part_floats = 4 << 20;
    s.argmax_part_entries = 65536;
    s.bytes = s.attn_part_floats * 4 + s.argmax_part_entries * 8 + 64 * 8;
    if (hipMalloc(&s.base, (size_t)s.bytes) != hipSuccess)
        return cleanup(fail(AESIR_ERR_HIP, "hipMalloc of context scratch failed"));
    char *p = (char *)s.base;
    s.attn_part = (float *)p;
    p += s.attn_part_floats * 4;
    s.argmax_part = p;
    p += s.argmax_part_entries * 8;
    s.result = (int64_t *)p;
    if (hipMemsetAsync(s.base, 0, (size_t)s.bytes, ctx->stream) != hipSuccess)
        return cleanup(fail(AESIR_ERR_HIP, "hipMemsetAsync of context scratch failed"));
    if (hipHostMalloc((void **)&ctx->pinned_i64, 64 * sizeof(int64_t), hipHostMallocDefault) != hipSuccess)
        return cleanup(fail(AESIR_ERR_HIP, "hipHostMalloc failed"));
    if (hipEventCreate(&ctx->ev_start) != hipSuccess || hipEventCreate(&ctx->ev_stop) != hipSuccess)
        return cleanup(fail(AESIR_ERR_HIP, "hipEventCreate failed"));
    if (hipStreamSynchronize(ctx->stream) != hipSuccess)
        return cleanup(fail(AESIR_ERR_HIP, "hipStreamSynchronize failed"));
    *out = ctx;
    return AESIR_OK;
}

int32_t aesir_ctx_destroy(aesir_ctx *ctx) {
    if (!ctx) return AESIR_OK;
    if (ctx->live_models > 0)  // a model keeps pointers into this context
        return fail(AESIR_ERR_INVALID, "aesir_ctx_destroy: %lld model(s) still alive; destroy them first",
                    (long long)ctx->live_models);
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (auto &t : ctx->rope_tables) (void)hipFree(t.dev);
    sampler_release(ctx);
    blas_release(ctx);
    if (ctx->scratch.base) (void)hipFree(ctx->scratch.base);
    if (ctx->well_base) (void)hipFree(ctx->well_base);
    if (ctx->pinned_i64) (void)hipHostFree(ctx->pinned_i64);
    if (ctx->ev_start) (void)hipEventDestroy(ctx->ev_start);
    if (ctx->ev_stop) (void)hipEventDestroy(ctx->ev_stop);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return AESIR_OK;
}

int32_t aesir_ctx_synchronize(aesir_ctx *ctx) {
    AESIR_TRY(bind(ctx));
    AESIR_HIP_TRY(hipStreamSynchronize(ctx->stream));
    return AESIR_OK;
}

void *aesir_ctx_stream(aesir_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int32_t aesir_ctx_device_info(aesir_ctx *ctx, char *arch_out, int32_t arch_cap, int32_t *cu_count,
                              int64_t *hbm_bytes) {
    if (!ctx) return fail(AESIR_ERR_INVALID, "aesir: null context");
    if (arch_out && arch_cap > 0) std::snprintf(arch_out, (size_t)arch_cap, "%s", ctx->arch);
    if (cu_count) *cu_count = ctx->cu_count;
    if (hbm_bytes) *hbm_bytes = ctx->hbm_bytes;
    return AESIR_OK;
}

int32_t aesir_well_allocate(aesir_ctx *ctx, int64_t elements, void **dev_ptr) {
    if (!ctx || !dev_ptr) return fail(AESIR_ERR_INVALID, "aesir_well_allocate: null argument");
    if (elements <= 0) return fail(AESIR_ERR_INVALID, "MimirWell: allocation count must be positive");
    return well_alloc_bytes(ctx, elements * 2, dev_ptr);
}

int32_t aesir_well_reset(aesir_ctx *ctx, int64_t offset) {
    if (!ctx) return fail(AESIR_ERR_INVALID, "aesir: null context");
    if (offset < 0 || offset > ctx->well_offset) return fail(AESIR_ERR_INVALID, "MimirWell: invalid reset offset");
    ctx->well_offset = offset;
    return AESIR_OK;
}

int64_t aesir_well_offset(const aesir_ctx *ctx) { return ctx ? ctx->well_offset : -1; }
int64_t aesir_well_capacity(const aesir_ctx *ctx) { return ctx ? ctx->well_capacity : -1; }

int32_t aesir_memcpy_h2d(aesir_ctx *ctx, void *dev_dst, const void *host_src, int64_t bytes) {
    AESIR_TRY(bind(ctx));
    if (bytes < 0) return fail(AESIR_ERR_INVALID, "aesir_memcpy_h2d: negative size");
    if (bytes == 0) return AESIR_OK;
    // Synchronous with respect to the host buffer: pageable source memory may be reused at once.
    AESIR_HIP_TRY(hipMemcpyAsync(dev_dst, host_src, (size_t)bytes, hipMemcpyHostToDevice, ctx->stream));
    AESIR_HIP_TRY(hipStreamSynchronize(ctx->stream));
    return AESIR_OK;
}

int32_t aesir_memcpy_d2h(aesir_ctx *ctx, void *host_dst, const void *dev_src, int64_t bytes) {
    AESIR_TRY(bind(ctx));
    if (bytes < 0) return fail(AESIR_ERR_INVALID, "aesir_memcpy_d2h: negative size");
    if (bytes == 0) return AESIR_OK;
    AESIR_HIP_TRY(hipMemcpyAsync(host_dst, dev_src, (size_t)bytes, hipMemcpyDeviceToHost, ctx->stream));
    AESIR_HIP_TRY(hipStreamSynchronize(ctx->stream));
    return AESIR_OK;
}

int32_t aesir_memcpy_d2d(aesir_ctx *ctx, void *dev_dst, const void *dev_src, int64_t bytes) {
    AESIR_TRY(bind(ctx));
    if (bytes < 0) return fail(AESIR_ERR_INVALID, "aesir_memcpy_d2d: negative size");
    if (bytes == 0) return AESIR_OK;
    AESIR_HIP_TRY(hipMemcpyAsync(dev_dst, dev_src, (size_t)bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return AESIR_OK;
}

int32_t aesir_timer_start(aesir_ctx *ctx) {
    AESIR_TRY(bind(ctx));
    AESIR_HIP_TRY(hipEventRecord(ctx->ev_start, ctx->stream));
    ctx->timer_running = true;
    return AESIR_OK;
}

int32_t aesir_timer_stop(aesir_ctx *ctx, float *elapsed_ms) {
    AESIR_TRY(bind(ctx));
    if (!ctx->timer_running) return fail(AESIR_ERR_INVALID, "aesir_timer_stop: timer not started");
    AESIR_HIP_TRY(hipEventRecord(ctx->ev_stop, ctx->stream));
    AESIR_HIP_TRY(hipEventSynchronize(ctx->ev_stop));
    AESIR_HIP_TRY(hipEventElapsedTime(elapsed_ms, ctx->ev_start, ctx->ev_stop));
    ctx->timer_running = false;
    return AESIR_OK;
}

}  // extern "C"
