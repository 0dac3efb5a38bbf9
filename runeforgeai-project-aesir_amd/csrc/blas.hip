// Prefill GEMMs of many rows on hipBLASLt (the batched path of gemm_f16, compute.mojo:1751-1854).
//
// At a chunk of hundreds of rows a prefill GEMM is matrix-core bound (1024 rows x 2048 K: 1024
// flop per weight byte, three times MI355X's ridge), which is where a library tile sized for that
// regime pays off; the hand-written wide-tile kernel stays for the short chunks, where the weight
// stream bounds it. The product is plain: D = A W^T with A [M][K] row-major f16 activations, W
// [N][K] row-major f16 weights, f32 accumulation and one rounding of each output, to f16 or to
// f32 for a row kernel that applies the rounding of the epilogue itself. Every epilogue of the
// prefill (SwiGLU, residual add, RMSNorm) stays a hand-written row kernel, so the rounding
// points are the fused kernels' own.
//
// In hipBLASLt's column-major terms D^T [N][M] = op(W) A^T with op = transpose on W stored as
// K x N (leading dimension K), A^T as K x M (leading dimension K) and D^T as N x M (leading
// dimension N, i.e. row-major [M][N]). The algorithm is the library heuristic's first choice for
// the shape (deterministic for a given library and device), cached per context with its
// descriptors.
#include <hipblaslt/hipblaslt.h>

#include <vector>

#include "kernels.hpp"

namespace aesir {

namespace {

struct BlasPlan {
    int64_t M = 0, N = 0, K = 0;
    bool f32_out = false;
    bool ok = false;
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, ld = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t ws = 0;
};

constexpr size_t kMaxPlans = 256;

struct BlasState {
    hipblasLtHandle_t handle = nullptr;
    std::vector<BlasPlan> plans;
};

void destroy_plan(BlasPlan &p) {
    if (p.la) (void)hipblasLtMatrixLayoutDestroy(p.la);
    if (p.lb) (void)hipblasLtMatrixLayoutDestroy(p.lb);
    if (p.ld) (void)hipblasLtMatrixLayoutDestroy(p.ld);
    if (p.desc) (void)hipblasLtMatmulDescDestroy(p.desc);
    p = BlasPlan{};
}

// Builds the descriptors and picks the algorithm for one shape; p.ok stays false when the library
// offers none within the workspace.
void make_plan(hipblasLtHandle_t h, BlasPlan &p, size_t ws_bytes) {
    const hipDataType dt = p.f32_out ? HIP_R_32F : HIP_R_16F;
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16F, p.K, p.N, p.K) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16F, p.K, p.M, p.K) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.ld, dt, p.N, p.M, p.N) != HIPBLAS_STATUS_SUCCESS)
        return;
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return;
    const uint64_t wsl = ws_bytes;
    hipblasLtMatmulHeuristicResult_t res[1];
    int n = 0;
    const bool got = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsl,
                                                           sizeof(wsl)) == HIPBLAS_STATUS_SUCCESS &&
                     hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.la, p.lb, p.ld, p.ld, pref, 1, res, &n) ==
                         HIPBLAS_STATUS_SUCCESS &&
                     n > 0 && res[0].state == HIPBLAS_STATUS_SUCCESS && res[0].workspaceSize <= ws_bytes;
    (void)hipblasLtMatmulPreferenceDestroy(pref);
    if (!got) return;
    p.algo = res[0].algo;
    p.ws = res[0].workspaceSize;
    p.ok = true;
}

}  // namespace

int32_t blas_gemm_nt(aesir_ctx *ctx, hipStream_t s, const void *A, int64_t M, int64_t K, const void *W, int64_t N,
                     void *D, bool f32_out, void *ws, int64_t ws_bytes) {
    if (M <= 0 || N <= 0 || K <= 0) return fail(AESIR_ERR_INVALID, "blas_gemm_nt: empty shape");
    if (!ctx->blas) {
        auto *st = new BlasState;
        if (hipblasLtCreate(&st->handle) != HIPBLAS_STATUS_SUCCESS) {
            delete st;
            return fail(AESIR_ERR_UNSUPPORTED, "hipblasLtCreate failed");
        }
        ctx->blas = st;
    }
    auto *st = static_cast<BlasState *>(ctx->blas);
    BlasPlan *plan = nullptr;
    for (BlasPlan &p : st->plans)
        if (p.M == M && p.N == N && p.K == K && p.f32_out == f32_out) plan = &p;
    if (!plan) {
        // every distinct chunk length brings its shapes: keep the most recent kMaxPlans
        if (st->plans.size() >= kMaxPlans) {
            destroy_plan(st->plans.front());
            st->plans.erase(st->plans.begin());
        }
        BlasPlan p;
        p.M = M, p.N = N, p.K = K, p.f32_out = f32_out;
        make_plan(st->handle, p, (size_t)ws_bytes);
        st->plans.push_back(p);
        plan = &st->plans.back();
    }
    if (!plan->ok) return fail(AESIR_ERR_UNSUPPORTED, "hipBLASLt offers no algorithm for %lld x %lld x %lld",
                               (long long)M, (long long)N, (long long)K);
    const float alpha = 1.0f, beta = 0.0f;
    if (hipblasLtMatmul(st->handle, plan->desc, &alpha, W, plan->la, A, plan->lb, &beta, D, plan->ld, D, plan->ld,
                        &plan->algo, plan->ws ? ws : nullptr, plan->ws, s) != HIPBLAS_STATUS_SUCCESS)
        return fail(AESIR_ERR_HIP, "hipblasLtMatmul failed (%lld x %lld x %lld)", (long long)M, (long long)N,
                    (long long)K);
    return AESIR_OK;
}

void blas_release(aesir_ctx *ctx) {
    auto *st = static_cast<BlasState *>(ctx->blas);
    if (!st) return;
    for (BlasPlan &p : st->plans) destroy_plan(p);
    if (st->handle) (void)hipblasLtDestroy(st->handle);
    delete st;
    ctx->blas = nullptr;
}

}  // namespace aesir
