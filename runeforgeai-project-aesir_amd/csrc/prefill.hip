// Batched prefill for gfx950: the prompt's positions go through each layer together, as M-row
// GEMMs on the matrix cores, instead of one forward_pass per position (the reference's
// _run_generation prefills by position, aesir.mojo:358-374; the result is the same KV cache and
// the same next token up to f32 summation order).
//
// MFMA GEMM  C[M][N] = A[M][K] . B[N][K]^T, f16 in, f32 accumulate (v_mfma_f32_16x16x32_f16).
//   A (activations) and B (weights) are both K-contiguous, so every MFMA operand fragment is one
//   16-byte row load: lane l holds row (l % 16) and k = 8 (l / 16) .. +7 of its 16 x 32 slice, the
//   same k order for A and B. A workgroup is 4 waves; wave w owns 16 weight rows (output
//   columns) and all 128 rows of its M tile, i.e. 8 accumulator tiles (rows 16i + 4 (l / 16) + e,
//   column l % 16 in lane l). The 4 waves read the same A fragments (the activation tile stays in
//   L1/L2) while each streams its own weight rows from HBM exactly once, one 32-wide k step ahead
//   of the MFMAs. At M = 128 the GEMM is HBM-bound (128 flop/byte against MI355X's 312 flop/byte
//   ridge), so the design favours streaming the weights over LDS tiling of A.
#include <cmath>
#include <vector>

#include "common.hpp"
#include "device.hpp"
#include "kernels.hpp"
#include "model.hpp"

namespace aesir {

typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));

constexpr int kGemmMT = 128;  // rows of A per workgroup tile
constexpr int kGemmWaves = 4;
constexpr int kGemmNW = 16;   // output columns per wave
constexpr int kGemmNT = kGemmWaves * kGemmNW;

enum GemmEpi : int { kEpiStore = 0, kEpiResidual = 1, kEpiSwiglu = 2 };

__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h16x8, a), __builtin_bit_cast(h16x8, b), c, 0, 0,
                                                  0);
}

// EPI: kEpiStore C[m][n] = f16(acc); kEpiResidual C[m][n] = f16(f16(acc) + C[m][n]);
// kEpiSwiglu with interleaved gate/up columns (2i gate, 2i + 1 up): C[m][i] = f16(up * silu(gate)).
// Requires K % 32 == 0 and 16-byte aligned rows (checked by the launcher).
template <int EPI>
__global__ __launch_bounds__(kGemmWaves * kWave) void gemm_mfma_kernel(const h16 *__restrict__ A, int64_t M,
                                                                       int64_t K, const h16 *__restrict__ B, int64_t N,
                                                                       h16 *__restrict__ C, int64_t ldc) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t m0 = (int64_t)blockIdx.y * kGemmMT;
    const int64_t n0 = ((int64_t)blockIdx.x * kGemmWaves + wave) * kGemmNW;
    if (n0 >= N) return;  // no workgroup-wide synchronization below
    const int r = lane & 15, g = lane >> 4;
    const h16 *ap[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int64_t m = m0 + 16 * i + r;
        ap[i] = A + (m < M ? m : M - 1) * K + 8 * g;  // rows past M re-read row M - 1, never stored
    }
    const h16 *bp = B + (n0 + r < N ? n0 + r : N - 1) * K + 8 * g;

    f32x4 acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    u32x4 a0[8], a1[8], b0, b1;
    auto load = [&](u32x4 (&a)[8], u32x4 &b, int64_t k) {
        b = ld16_stream(bp + k);
#pragma unroll
        for (int i = 0; i < 8; i++) a[i] = ld16(ap[i] + k);
    };
    auto mma = [&](const u32x4 (&a)[8], u32x4 b) {
#pragma unroll
        for (int i = 0; i < 8; i++) acc[i] = mfma16x16x32(a[i], b, acc[i]);
    };
    load(a0, b0, 0);
    for (int64_t k = 0; k < K; k += 64) {
        const bool two = k + 32 < K;
        if (two) load(a1, b1, k + 32);
        mma(a0, b0);
        if (!two) break;
        if (k + 64 < K) load(a0, b0, k + 64);
        mma(a1, b1);
    }

    const int64_t n = n0 + r;
#pragma unroll
    for (int i = 0; i < 8; i++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int64_t m = m0 + 16 * i + 4 * g + e;
            const float v = acc[i][e];
            if (EPI == kEpiSwiglu) {
                const float up = __shfl_xor(v, 1, kWave);  // lane r ^ 1 holds column n ^ 1
                if ((r & 1) == 0 && m < M && n + 1 < N)
                    C[m * ldc + n / 2] = hmul((h16)up, silu_h((h16)v));
            } else if (m < M && n < N) {
                h16 *c = C + m * ldc + n;
                *c = EPI == kEpiResidual ? hadd((h16)v, *c) : (h16)v;
            }
        }
    }
}

static bool mfma_shape_ok(const void *A, int64_t K, const void *B) {
    return K % 32 == 0 && ((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0;
}

template <int EPI>
static int32_t launch_mfma(hipStream_t s, const void *A, int64_t M, int64_t K, const void *B, int64_t N, void *C,
                           int64_t ldc, const char *name) {
    const int64_t gx = (N + kGemmNT - 1) / kGemmNT, gy = (M + kGemmMT - 1) / kGemmMT;
    if (gx > 2147483647 || gy > 65535) return fail(AESIR_ERR_UNSUPPORTED, "%s: GEMM grid too large", name);
    hipLaunchKernelGGL(gemm_mfma_kernel<EPI>, dim3((unsigned)gx, (unsigned)gy), dim3(kGemmWaves * kWave), 0, s,
                       (const h16 *)A, M, K, (const h16 *)B, N, (h16 *)C, ldc);
    AESIR_LAUNCH_CHECK(name);
    return AESIR_OK;
}

int32_t launch_gemm_f16_mfma(aesir_ctx *ctx, const void *A, int64_t M, int64_t K, const void *B, int64_t N, void *C) {
    if (!mfma_shape_ok(A, K, B)) return launch_gemm_f16(ctx, A, M, K, B, N, C);
    return launch_mfma<kEpiStore>(ctx->stream, A, M, K, B, N, C, N, "gemm_mfma_kernel");
}

// ------------------------------------------------------------------ row kernels of the prefill

// Y[r] = rmsnorm(X[r]) out of place, one workgroup per row (compute.mojo:2178-2204).
constexpr int kPThreads = 256;
__global__ __launch_bounds__(kPThreads) void rmsnorm_rows_kernel(const h16 *__restrict__ X, h16 *__restrict__ Y,
                                                                 int64_t cols, const h16 *__restrict__ w, float eps) {
    __shared__ float red[kPThreads / kWave];
    const h16 *x = X + (int64_t)blockIdx.x * cols;
    h16 *y = Y + (int64_t)blockIdx.x * cols;
    float ss = 0.0f;
    for (int64_t c = threadIdx.x; c < cols; c += kPThreads) {
        const float v = (float)x[c];
        ss = fmaf(v, v, ss);
    }
    ss = block_sum<kPThreads / kWave>(ss, red);
    const h16 inv = (h16)(1.0f / sqrtf(ss / (float)cols + eps));
    for (int64_t c = threadIdx.x; c < cols; c += kPThreads) y[c] = hmul(hmul(x[c], inv), w[c]);
}

// X[r] = token_embd[tokens[r]] (inference.mojo:452-467), one workgroup per row.
__global__ __launch_bounds__(kPThreads) void embed_rows_kernel(const h16 *__restrict__ table, int64_t dim,
                                                               const int64_t *__restrict__ tokens, h16 *__restrict__ X) {
    const h16 *src = table + tokens[blockIdx.x] * dim;
    h16 *dst = X + (int64_t)blockIdx.x * dim;
    for (int64_t c = threadIdx.x; c < dim; c += kPThreads) dst[c] = src[c];
}

// Row r of QKV [M][dim + 2 kvd] at position p0 + r: RoPE on its Q and K pairs (apply_rope,
// compute.mojo:2232-2244, cos/sin from the host-built table) into Q [M][dim] and the K cache slot,
// V copied to the V cache slot (KVCache.append at pos % max_seq, mimir_well.mojo:488-501).
__global__ __launch_bounds__(kPThreads) void qkv_post_rows_kernel(const h16 *__restrict__ qkv, int64_t dim,
                                                                  int64_t kvd, int64_t hd, int64_t p0, int64_t max_seq,
                                                                  const h16x2 *__restrict__ rope, h16 *__restrict__ Q,
                                                                  h16 *__restrict__ kc, h16 *__restrict__ vc) {
    const int64_t r = blockIdx.x, pos = p0 + r, slot = pos % max_seq;
    const h16 *row = qkv + r * (dim + 2 * kvd);
    const int64_t pairs = (dim + kvd) / 2;
    for (int64_t j = threadIdx.x; j < pairs + kvd / 2; j += kPThreads) {
        const int64_t col = 2 * j;
        const h16 a = row[col], b = row[col + 1];
        if (j < pairs) {
            const int64_t c = col < dim ? col : col - dim;
            const h16x2 cs = rope[pos * (hd / 2) + ((c % hd) >> 1)];
            h16 *dst = col < dim ? Q + r * dim + c : kc + slot * kvd + c;
            dst[0] = hsub(hmul(a, cs.x), hmul(b, cs.y));
            dst[1] = hadd(hmul(a, cs.y), hmul(b, cs.x));
        } else {
            h16 *dst = vc + slot * kvd + (col - dim - kvd);
            dst[0] = a;
            dst[1] = b;
        }
    }
}

// Causal GQA attention of the prefill rows: query row r (position p0 + r) of head h attends to
// positions [0, min(p0 + r + 1, max_seq)) of the layer's cache, which already holds this chunk's
// K/V rows. One wave per (row, head): 64 positions per round (one per lane, q . k in f32), f32
// online softmax with wave reductions, then each lane accumulates the head dims lane, lane + 64,
// ... over the round's positions. Same arithmetic as flash_attention_gqa (compute.mojo:1950-2015)
// with an f32 accumulator.
constexpr int kMaxHdPerLane = 4;  // head_dim <= 256
__global__ __launch_bounds__(kWave) void prefill_attention_kernel(const h16 *__restrict__ Q, const h16 *__restrict__ kc,
                                                                  const h16 *__restrict__ vc, h16 *__restrict__ out,
                                                                  int64_t dim, int64_t kvd, int64_t hd, int64_t G,
                                                                  int64_t p0, int64_t max_seq, float scale) {
    __shared__ float qs[256];
    __shared__ float ps[kWave];
    const int lane = threadIdx.x;
    const int64_t r = blockIdx.x, h = blockIdx.y, g = h / G;
    const int64_t pos = p0 + r;
    const int64_t S = pos + 1 < max_seq ? pos + 1 : max_seq;
    const h16 *q = Q + r * dim + h * hd;
    for (int64_t d = lane; d < hd; d += kWave) qs[d] = (float)q[d];
    __syncthreads();
    const h16 *Kg = kc + g * hd;
    const h16 *Vg = vc + g * hd;
    float m = -INFINITY, l = 0.0f, acc[kMaxHdPerLane];
#pragma unroll
    for (int j = 0; j < kMaxHdPerLane; j++) acc[j] = 0.0f;
    for (int64_t c0 = 0; c0 < S; c0 += kWave) {
        const int64_t p = c0 + lane;
        float s = -INFINITY;
        if (p < S) {
            const h16 *k = Kg + p * kvd;
            float d = 0.0f;
            for (int64_t i = 0; i < hd; i++) d = fmaf(qs[i], (float)k[i], d);
            s = d * scale;
        }
        const float mn = fmaxf(m, wave_max(s));
        const float pr = p < S ? expf(s - mn) : 0.0f;
        const float al = expf(m - mn);  // 0 on the first round
        l = l * al + wave_sum(pr);
        m = mn;
        __syncthreads();
        ps[lane] = pr;
        __syncthreads();
        const int64_t n = S - c0 < kWave ? S - c0 : kWave;
#pragma unroll
        for (int j = 0; j < kMaxHdPerLane; j++) {
            const int64_t d = lane + kWave * j;
            if (d >= hd) continue;
            float a = acc[j] * al;
            for (int64_t t = 0; t < n; t++) a = fmaf(ps[t], (float)Vg[(c0 + t) * kvd + d], a);
            acc[j] = a;
        }
    }
    h16 *o = out + r * dim + h * hd;
#pragma unroll
    for (int j = 0; j < kMaxHdPerLane; j++) {
        const int64_t d = lane + kWave * j;
        if (d < hd) o[d] = (h16)(acc[j] / l);
    }
}

// act[i] = f16(up * silu(gate)) over interleaved [gate, up] pairs gu[2i], gu[2i + 1]
// (inference.mojo:257-260 on the gate/up GEMM rows as this build lays them out).
__global__ __launch_bounds__(kPThreads) void swiglu_pairs_kernel(const h16 *__restrict__ gu, h16 *__restrict__ act,
                                                                 int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kPThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kPThreads)
        act[i] = hmul(gu[2 * i + 1], silu_h(gu[2 * i]));
}

static int32_t launch_swiglu_pairs(hipStream_t s, const void *gu, void *act, int64_t n) {
    int64_t g = (n + kPThreads - 1) / kPThreads;
    if (g > 65536) g = 65536;
    hipLaunchKernelGGL(swiglu_pairs_kernel, dim3((unsigned)g), dim3(kPThreads), 0, s, (const h16 *)gu, (h16 *)act, n);
    AESIR_LAUNCH_CHECK("swiglu_pairs_kernel");
    return AESIR_OK;
}

// ------------------------------------------------------------------ the batched pass

// Runs positions [p0, p0 + n) of tokens through every layer (n <= the model's prefill rows).
static int32_t prefill_chunk(aesir_model *m, const int64_t *tokens_host, int64_t p0, int64_t n) {
    const aesir_model_config &c = m->cfg;
    hipStream_t s = m->ctx->stream;
    const int64_t d = c.dim, kvd = m->kvd, f = c.ffn, hd = m->hd;
    const int64_t qkv_n = d + 2 * kvd;
    h16 *X = (h16 *)m->pf_x, *Xn = (h16 *)m->pf_xn, *QKV = (h16 *)m->pf_qkv, *Q = (h16 *)m->pf_q;
    h16 *ATT = (h16 *)m->pf_att, *ACT = (h16 *)m->pf_act;
    AESIR_HIP_TRY(hipMemcpyAsync(m->pf_tokens, tokens_host, (size_t)n * sizeof(int64_t), hipMemcpyHostToDevice, s));
    hipLaunchKernelGGL(embed_rows_kernel, dim3((unsigned)n), dim3(kPThreads), 0, s, (const h16 *)m->tok_embd, d,
                       (const int64_t *)m->pf_tokens, X);
    AESIR_LAUNCH_CHECK("embed_rows_kernel");
    const bool mfma = d % 32 == 0 && f % 32 == 0;
    for (int64_t l = 0; l < c.n_layers; l++) {
        const ModelLayer &L = m->layers[l];
        h16 *kc = (h16 *)m->k_cache + l * c.ctx_len * kvd, *vc = (h16 *)m->v_cache + l * c.ctx_len * kvd;
        // attention block (inference.mojo:166-232)
        hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3((unsigned)n), dim3(kPThreads), 0, s, X, Xn, d,
                           (const h16 *)L.attn_norm, c.rms_eps);
        AESIR_LAUNCH_CHECK("rmsnorm_rows_kernel");
        if (mfma) AESIR_TRY(launch_mfma<kEpiStore>(s, Xn, n, d, L.wqkv, qkv_n, QKV, qkv_n, "gemm_mfma_qkv"));
        else AESIR_TRY(launch_gemm_f16(m->ctx, Xn, n, d, L.wqkv, qkv_n, QKV));
        hipLaunchKernelGGL(qkv_post_rows_kernel, dim3((unsigned)n), dim3(kPThreads), 0, s, QKV, d, kvd, hd, p0,
                           c.ctx_len, (const h16x2 *)m->rope, Q, kc, vc);
        AESIR_LAUNCH_CHECK("qkv_post_rows_kernel");
        hipLaunchKernelGGL(prefill_attention_kernel, dim3((unsigned)n, (unsigned)c.n_heads), dim3(kWave), 0, s, Q, kc,
                           vc, ATT, d, kvd, hd, c.n_heads / c.n_kv_heads, p0, c.ctx_len, m->attn_scale);
        AESIR_LAUNCH_CHECK("prefill_attention_kernel");
        if (mfma) {
            AESIR_TRY(launch_mfma<kEpiResidual>(s, ATT, n, d, L.wo, d, X, d, "gemm_mfma_o_residual"));
        } else {
            AESIR_TRY(launch_gemm_f16(m->ctx, ATT, n, d, L.wo, d, Xn));
            AESIR_TRY(launch_residual_add(s, X, Xn, n * d));
        }
        // feed-forward block (inference.mojo:235-273)
        hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3((unsigned)n), dim3(kPThreads), 0, s, X, Xn, d,
                           (const h16 *)L.ffn_norm, c.rms_eps);
        AESIR_LAUNCH_CHECK("rmsnorm_rows_kernel");
        if (mfma) {
            AESIR_TRY(launch_mfma<kEpiSwiglu>(s, Xn, n, d, L.wgu, 2 * f, ACT, f, "gemm_mfma_gate_up_swiglu"));
            AESIR_TRY(launch_mfma<kEpiResidual>(s, ACT, n, f, L.wdown, d, X, d, "gemm_mfma_down_residual"));
        } else {
            // interleaved gate/up rows -> [n][2f] products, then the SwiGLU over the pairs
            AESIR_TRY(launch_gemm_f16(m->ctx, Xn, n, d, L.wgu, 2 * f, m->pf_gu));
            AESIR_TRY(launch_swiglu_pairs(s, m->pf_gu, ACT, n * f));
            AESIR_TRY(launch_gemm_f16(m->ctx, ACT, n, f, L.wdown, d, Xn));
            AESIR_TRY(launch_residual_add(s, X, Xn, n * d));
        }
    }
    return AESIR_OK;
}

int32_t model_prefill(aesir_model *m, const int64_t *tokens, int64_t n, int64_t start_pos, int64_t *next) {
    const aesir_model_config &c = m->cfg;
    if (n <= 0) {
        *next = 0;
        return AESIR_OK;
    }
    if (start_pos < 0) return fail(AESIR_ERR_INVALID, "apply_rope: start_pos cannot be negative");
    for (int64_t i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= c.vocab)
            return fail(AESIR_ERR_INVALID, "Prompt token ID is outside the embedding vocabulary");
    AESIR_TRY(ensure_rope(m, start_pos + n));
    for (int64_t r0 = 0; r0 < n; r0 += m->pf_rows) {
        const int64_t rows = n - r0 < m->pf_rows ? n - r0 : m->pf_rows;
        AESIR_TRY(prefill_chunk(m, tokens + r0, start_pos + r0, rows));
    }
    // last position: output norm, lm_head and greedy argmax on the decode path's kernels
    const int64_t last = (n - 1) % m->pf_rows;
    hipStream_t s = m->ctx->stream;
    AESIR_HIP_TRY(hipMemcpyAsync(m->x, (h16 *)m->pf_x + last * c.dim, (size_t)c.dim * 2, hipMemcpyDeviceToDevice, s));
    AESIR_TRY(upload_state(m, tokens[n - 1], start_pos + n - 1, 0, m->ring_cap));
    AESIR_TRY(launch_lm_head_argmax(s, lm_args(m, false)));
    AESIR_HIP_TRY(hipMemcpyAsync(m->state_host, m->state, sizeof(DecodeState), hipMemcpyDeviceToHost, s));
    AESIR_HIP_TRY(hipStreamSynchronize(s));
    *next = m->state_host->next_token;
    return AESIR_OK;
}

}  // namespace aesir

using namespace aesir;

extern "C" int32_t aesir_prefill(aesir_model *m, const int64_t *tokens, int64_t n_tokens, int64_t start_pos,
                                 int64_t *next_token) {
    if (!m || !next_token) return fail(AESIR_ERR_INVALID, "aesir_prefill: null argument");
    if (n_tokens > 0 && !tokens) return fail(AESIR_ERR_INVALID, "aesir_prefill: null token list");
    AESIR_TRY(bind(m->ctx));
    if (start_pos + n_tokens > m->cfg.ctx_len)
        return fail(AESIR_ERR_INVALID, "Prompt token count exceeds the model context length");
    return model_prefill(m, tokens, n_tokens, start_pos, next_token);
}
