// Prefill: M > 1 GEMM and the batched prompt path.
#include "common.hpp"
#include "kernels.hpp"
#include "model.hpp"

namespace aesir {

int32_t launch_gemm_f16_mfma(aesir_ctx *ctx, const void *A, int64_t M, int64_t K, const void *B, int64_t N, void *C) {
    return launch_gemm_f16(ctx, A, M, K, B, N, C);
}

int32_t model_prefill(aesir_model *m, const int64_t *tokens, int64_t n, int64_t *next) {
    for (int64_t p = 0; p < n; p++) AESIR_TRY(aesir_forward_pass(m, tokens, n, p, next));
    return AESIR_OK;
}

}  // namespace aesir
