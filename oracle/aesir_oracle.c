/*
 * aesir_oracle.c -- CPU restatement of A.E.S.I.R.'s verified Llama F16 forward path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or shipped): loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg. Single-threaded, like the
 * reference (which has no parallelize anywhere).
 *
 * Citations are to the reference repository (paths under aesir_engine/).
 *
 * Arithmetic conventions that the reference fixes:
 *   - binary16 storage after every op, round-to-nearest-even (Mojo .cast[f16]()).
 *   - f16 x f16 -> f16 ops (RMSNorm scale, RoPE rotation, SiLU, SwiGLU mul, residual add) are
 *     evaluated in f32 and rounded once to f16. For +, -, *, / this equals the correctly rounded
 *     binary16 result (24 >= 2*11+2, so the double rounding is innocuous).
 *   - No floating-point contraction anywhere (built with -ffp-contract=off).
 *   - The 16-lane SIMD reduce_add of the reference (simd_w_f16 = 16, compute.mojo:19-20) is
 *     evaluated as a halving tree: lanes i and i+8, then i and i+4, i and i+2, then 0 and 1.
 *     That lane order is Mojo-stdlib behaviour that this repository cannot run; it is
 *     documented as the unpinned last bit of gemm_f16 and rmsnorm.
 */
#include "aesir_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#define AO_HAVE_X86 1
#else
#define AO_HAVE_X86 0
#endif

static __thread char g_err[512];

static int ao_fail(int code, const char *msg) {
    snprintf(g_err, sizeof g_err, "%s", msg);
    return code;
}

const char *ao_last_error(void) { return g_err; }

/* ------------------------------------------------------------------ binary16 */

uint16_t ao_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) {
        if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu)); /* quiet NaN */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to infinity */
    if (a < 0x38800000u) {                                   /* below 2^-14: subnormal or zero */
        if (a < 0x33000000u) return (uint16_t)sign;          /* below 2^-25 rounds to zero */
        uint32_t e = a >> 23;
        uint32_t m = (a & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* value / 2^-24 = m * 2^(e-126) */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = ((a >> 23) - 112u) << 10 | ((a >> 13) & 0x3ffu);
    uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

float ao_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else { /* subnormal: m * 2^-24 is exact in f32 */
            float v = (float)m * 5.9604644775390625e-08f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

void ao_f32_to_f16_array(const float *src, uint16_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = ao_f32_to_f16(src[i]);
}

void ao_f16_to_f32_array(const uint16_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = ao_f16_to_f32(src[i]);
}

#define H2F(h) ao_f16_to_f32(h)
#define F2H(f) ao_f32_to_f16(f)

/* f16 op f16 -> f16, one rounding (see header note). */
static inline uint16_t hmul(uint16_t a, uint16_t b) { return F2H(H2F(a) * H2F(b)); }
static inline uint16_t hadd(uint16_t a, uint16_t b) { return F2H(H2F(a) + H2F(b)); }
static inline uint16_t hsub(uint16_t a, uint16_t b) { return F2H(H2F(a) - H2F(b)); }
static inline uint16_t hdiv(uint16_t a, uint16_t b) { return F2H(H2F(a) / H2F(b)); }

/* ------------------------------------------------- 16-lane chunk dot products */

/* One simd_w_f16 = 16 chunk: products in f32 (exact for f16 inputs), then the halving tree. */
static float chunk16_dot_scalar(const uint16_t *a, const uint16_t *b) {
    float p[16];
    for (int i = 0; i < 16; i++) p[i] = H2F(a[i]) * H2F(b[i]);
    float s8[8], s4[4], s2[2];
    for (int i = 0; i < 8; i++) s8[i] = p[i] + p[i + 8];
    for (int i = 0; i < 4; i++) s4[i] = s8[i] + s8[i + 4];
    for (int i = 0; i < 2; i++) s2[i] = s4[i] + s4[i + 2];
    return s2[0] + s2[1];
}

#if AO_HAVE_X86
__attribute__((target("avx2,f16c"))) static float dot_f16_avx2(const uint16_t *a, const uint16_t *b, int64_t n16,
                                                              float sum) {
    for (int64_t c = 0; c < n16; c += 16) {
        __m256 a0 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(a + c)));
        __m256 a1 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(a + c + 8)));
        __m256 b0 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(b + c)));
        __m256 b1 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(b + c + 8)));
        __m256 s8 = _mm256_add_ps(_mm256_mul_ps(a0, b0), _mm256_mul_ps(a1, b1));
        __m128 s4 = _mm_add_ps(_mm256_castps256_ps128(s8), _mm256_extractf128_ps(s8, 1));
        __m128 s2 = _mm_add_ps(s4, _mm_movehl_ps(s4, s4));
        __m128 s1 = _mm_add_ss(s2, _mm_shuffle_ps(s2, s2, 1));
        sum += _mm_cvtss_f32(s1);
    }
    return sum;
}
static int g_simd = -1;
static int simd_ok(void) {
    if (g_simd < 0) g_simd = (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("f16c")) ? 1 : 0;
    return g_simd;
}
#else
static int simd_ok(void) { return 0; }
#endif

int ao_simd_enabled(void) { return simd_ok(); }

/* Sum over the 16-lane chunks of a.b, in chunk order, starting from `sum`. */
static float dot_chunks(const uint16_t *a, const uint16_t *b, int64_t n16, float sum) {
#if AO_HAVE_X86
    if (simd_ok()) return dot_f16_avx2(a, b, n16, sum);
#endif
    for (int64_t c = 0; c < n16; c += 16) sum += chunk16_dot_scalar(a + c, b + c);
    return sum;
}

/* ------------------------------------------------------------------ kernels */

/* gemm_f16, compute.mojo:1751-1854 (dense F16 loop :1831-1854). C[m,n] = f16(sum_k A[m,k]*B[n,k]). */
int ao_gemm_f16(const uint16_t *A, int64_t a_rows, int64_t a_cols, const uint16_t *B, int64_t b_rows,
                int64_t b_cols, uint16_t *C, int64_t c_rows, int64_t c_cols) {
    if (a_rows <= 0 || a_cols <= 0 || b_rows <= 0 || b_cols <= 0)
        return ao_fail(AO_ERR_INVALID, "gemm_f16: matrix dimensions must be positive");
    if (a_cols != b_cols) return ao_fail(AO_ERR_SHAPE, "gemm_f16: inner matrix dimension mismatch");
    if (c_rows != a_rows || c_cols != b_rows) return ao_fail(AO_ERR_SHAPE, "gemm_f16: output matrix shape mismatch");
    const int64_t K = a_cols;
    const int64_t simd_end = (K / 16) * 16;
    for (int64_t row = 0; row < a_rows; row++) {
        const uint16_t *a = A + row * K;
        for (int64_t n = 0; n < b_rows; n++) {
            const uint16_t *b = B + n * K;
            float sum = dot_chunks(a, b, simd_end, 0.0f);
            for (int64_t k = simd_end; k < K; k++) sum += H2F(a[k]) * H2F(b[k]); /* scalar tail :1847-1853 */
            C[row * b_rows + n] = F2H(sum);
        }
    }
    return AO_OK;
}

/* rmsnorm, compute.mojo:2166-2204. In place; inv_rms rounded to f16; two f16 roundings per element. */
int ao_rmsnorm_f16(uint16_t *T, int64_t rows, int64_t cols, const uint16_t *w, int64_t w_size, float eps) {
    if (rows <= 0 || cols <= 0) return ao_fail(AO_ERR_INVALID, "rmsnorm: tensor dimensions must be positive");
    if (w_size < cols) return ao_fail(AO_ERR_SHAPE, "rmsnorm: weight dimension mismatch");
    if (!(eps > 0.0f)) return ao_fail(AO_ERR_INVALID, "rmsnorm: epsilon must be positive");
    const int64_t simd_end = (cols / 16) * 16;
    for (int64_t r = 0; r < rows; r++) {
        uint16_t *x = T + r * cols;
        float ss = dot_chunks(x, x, simd_end, 0.0f);
        for (int64_t c = simd_end; c < cols; c++) {
            float v = H2F(x[c]);
            ss += v * v;
        }
        float rms = sqrtf(ss / (float)cols + eps);
        uint16_t inv_rms = F2H(1.0f / rms);
        for (int64_t c = 0; c < cols; c++) x[c] = hmul(hmul(x[c], inv_rms), w[c]);
    }
    return AO_OK;
}

/* apply_rope, compute.mojo:2207-2244. Adjacent-pair rotation in f16 arithmetic; angle in f32. */
int ao_rope_f16(uint16_t *Q, int64_t q_rows, int64_t q_cols, uint16_t *K, int64_t k_rows, int64_t k_cols,
                int64_t start_pos, int64_t head_dim, float theta) {
    if (start_pos < 0) return ao_fail(AO_ERR_INVALID, "apply_rope: start_pos cannot be negative");
    if (head_dim <= 0 || head_dim % 2 != 0)
        return ao_fail(AO_ERR_INVALID, "apply_rope: head_dim must be positive and even");
    if (q_cols % head_dim != 0 || k_cols % head_dim != 0)
        return ao_fail(AO_ERR_SHAPE, "apply_rope: tensor columns must be a multiple of head_dim");
    if (q_rows <= 0 || k_rows <= 0) return ao_fail(AO_ERR_INVALID, "apply_rope: tensor dimensions must be positive");
    /* The reference indexes K with Q's row count; a shorter K would be written out of bounds. */
    if (k_rows < q_rows) return ao_fail(AO_ERR_SHAPE, "apply_rope: K rows must cover Q rows");
    const int64_t nq = q_cols / head_dim, nk = k_cols / head_dim;
    /* The reference loops over Q.rows only and indexes K with the same row (:2226-2244). */
    for (int64_t r = 0; r < q_rows; r++) {
        int64_t pos = start_pos + r;
        for (int64_t i = 0; i < head_dim; i += 2) {
            float freq = 1.0f / powf(theta, (float)i / (float)head_dim);
            float val = (float)pos * freq;
            uint16_t fcr = F2H(cosf(val));
            uint16_t fci = F2H(sinf(val));
            for (int64_t h = 0; h < nq; h++) {
                uint16_t *p = Q + r * q_cols + h * head_dim + i;
                uint16_t q0 = p[0], q1 = p[1];
                p[0] = hsub(hmul(q0, fcr), hmul(q1, fci));
                p[1] = hadd(hmul(q0, fci), hmul(q1, fcr));
            }
            for (int64_t h = 0; h < nk; h++) {
                uint16_t *p = K + r * k_cols + h * head_dim + i;
                uint16_t k0 = p[0], k1 = p[1];
                p[0] = hsub(hmul(k0, fcr), hmul(k1, fci));
                p[1] = hadd(hmul(k0, fci), hmul(k1, fcr));
            }
        }
    }
    return AO_OK;
}

/* flash_attention_gqa, compute.mojo:1950-2015. One query row; the output accumulator is stored as
 * f16 after every position (:1994-2004). Invalid inputs return with the output untouched. */
void ao_attn_gqa(const uint16_t *q, int64_t q_rows, const uint16_t *keys, int64_t keys_cols,
                 const uint16_t *values, int64_t values_cols, uint16_t *out, int64_t out_rows,
                 int64_t seq_len, int64_t head_dim, int64_t nq, int64_t nkv) {
    if (seq_len <= 0 || q_rows != 1 || out_rows != 1) return;
    if (nq <= 0 || nkv <= 0 || head_dim <= 0) return;
    if (nq % nkv != 0) return;
    const int64_t per_kv = nq / nkv;
    const float scale = (float)(1.0 / pow((double)head_dim, 0.5));
    for (int64_t h = 0; h < nq; h++) {
        const int64_t g = h / per_kv;
        const uint16_t *qh = q + h * head_dim;
        uint16_t *o = out + h * head_dim;
        for (int64_t d = 0; d < head_dim; d++) o[d] = 0;
        float running_max = -1e20f, running_sum = 0.0f;
        for (int64_t p = 0; p < seq_len; p++) {
            const uint16_t *kp = keys + p * keys_cols + g * head_dim;
            const uint16_t *vp = values + p * values_cols + g * head_dim;
            float score = 0.0f;
            for (int64_t d = 0; d < head_dim; d++) score += H2F(qh[d]) * H2F(kp[d]);
            score *= scale;
            float next_max = running_max > score ? running_max : score;
            float prev_scale = expf(running_max - next_max);
            float prob = expf(score - next_max);
            float next_sum = running_sum * prev_scale + prob;
            for (int64_t d = 0; d < head_dim; d++) {
                float prev = H2F(o[d]);
                o[d] = F2H(prev * prev_scale + prob * H2F(vp[d]));
            }
            running_max = next_max;
            running_sum = next_sum;
        }
        for (int64_t d = 0; d < head_dim; d++) o[d] = F2H(H2F(o[d]) / running_sum);
    }
}

/* silu, compute.mojo:2113-2126: x * (1 / (1 + exp(-x))) with every op in f16. Mojo's exp on f16
 * evaluates in f32 and rounds to f16; expf stands in for it here. */
void ao_silu_f16(uint16_t *T, int64_t size) {
    if (size <= 0) return;
    const uint16_t one = 0x3c00;
    for (int64_t i = 0; i < size; i++) {
        uint16_t x = T[i];
        uint16_t e = F2H(expf(-H2F(x)));
        uint16_t sig = hdiv(one, hadd(one, e));
        T[i] = hmul(x, sig);
    }
}

/* SwiGLU product, inference.mojo:257-260: up[i] = f16(up[i] * gate[i]). */
void ao_mul_f16(uint16_t *up, const uint16_t *gate, int64_t size) {
    for (int64_t i = 0; i < size; i++) up[i] = hmul(up[i], gate[i]);
}

/* Residual add, inference.mojo:230-232 and :271-273: x = f16(x + residual). */
void ao_residual_add_f16(uint16_t *x, const uint16_t *residual, int64_t size) {
    for (int64_t i = 0; i < size; i++) x[i] = hadd(x[i], residual[i]);
}

/* Argmax, inference.mojo:508-515: floor f16(-10000), strict '>', first maximal index wins,
 * NaN never selected, 0 when nothing exceeds the floor. */
int64_t ao_argmax_f16(const uint16_t *logits, int64_t n) {
    float max_val = H2F(F2H(-10000.0f));
    int64_t best = 0;
    for (int64_t i = 0; i < n; i++) {
        float v = H2F(logits[i]);
        if (v > max_val) {
            max_val = v;
            best = i;
        }
    }
    return best;
}

/* sanitize_logit, sampler.mojo:9-14 */
static float sanitize_logit(float v) { return (isnan(v) || isinf(v)) ? -1e9f : v; }

/* Greedy branch of sample_token_from_logits, sampler.mojo:241-261. */
int64_t ao_greedy_sample_f16(const uint16_t *logits, int64_t n, const int64_t *suppress, int64_t n_suppress) {
    if (n <= 0) return 0;
    int64_t best = 0;
    float max_val = sanitize_logit(H2F(logits[0]));
    for (int64_t s = 0; s < n_suppress; s++)
        if (suppress[s] == 0) {
            max_val = -1e9f;
            break;
        }
    for (int64_t i = 1; i < n; i++) {
        float v = sanitize_logit(H2F(logits[i]));
        for (int64_t s = 0; s < n_suppress; s++)
            if (suppress[s] == i) {
                v = -1e9f;
                break;
            }
        if (v > max_val) {
            max_val = v;
            best = i;
        }
    }
    return best;
}

/* ---- full sampler stack, sampler.mojo:17-305 -------------------------------------------- */

/* RuneRNG.next_float32, sampler.mojo:39-42: uniform in [0, 1) from the low 24 bits. */
float ao_rune_rng_next_float32(uint64_t *state) {
    uint64_t v = ao_rune_rng_next(state);
    return (float)(v & 0xFFFFFFULL) / 16777216.0f;
}

/* f32 exp of the sampler stages. The reference calls Mojo's f32 exp; this restatement uses the
 * correctly rounded value (exp in f64, rounded once), which the GPU sampler computes the same way. */
static float exp_f32(float x) { return (float)exp((double)x); }

typedef struct {
    int64_t id;
    float logit;
} cand_t;

/* Order of sort_candidates_descending (sampler.mojo:92-104), a stable insertion sort on the
 * logit: descending logits, equal logits (-0 == +0) in their original order. Every sort of the
 * stack starts from index order or from an already sorted prefix, so the original order is the
 * id order and this total order gives the same permutation in O(n log n). */
static int cand_cmp(const void *pa, const void *pb) {
    const cand_t *a = (const cand_t *)pa, *b = (const cand_t *)pb;
    if (a->logit > b->logit) return -1;
    if (a->logit < b->logit) return 1;
    return a->id < b->id ? -1 : (a->id > b->id ? 1 : 0);
}

/* Softmax of the (sorted) candidate prefix as apply_top_p / apply_min_p compute it (:127-138,
 * :176-187): p = exp(l - l[0]) summed in order, then divided by the sum when it is positive. */
static void stage_probs(const cand_t *c, int64_t n, float *probs) {
    const float max_logit = c[0].logit;
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        probs[i] = exp_f32(c[i].logit - max_logit);
        sum += probs[i];
    }
    if (sum > 0.0f)
        for (int64_t i = 0; i < n; i++) probs[i] /= sum;
}

int64_t ao_sample_candidates_f16(const uint16_t *logits, int64_t vocab, const ao_sampler_config *cfg,
                                 const int64_t *context, int64_t n_context, const int64_t *suppress,
                                 int64_t n_suppress, int64_t *ids_out, float *logits_out) {
    if (vocab <= 0) return 0;
    cand_t *c = (cand_t *)malloc((size_t)vocab * sizeof(cand_t));
    int32_t *count = (int32_t *)calloc((size_t)vocab, sizeof(int32_t));
    float *probs = (float *)malloc((size_t)vocab * sizeof(float));
    for (int64_t i = 0; i < vocab; i++) {
        c[i].id = i;
        c[i].logit = sanitize_logit(H2F(logits[i]));
    }
    /* apply_token_mask (:197-211) */
    for (int64_t s = 0; s < n_suppress; s++)
        if (suppress[s] >= 0 && suppress[s] < vocab) c[suppress[s]].logit = -1e9f;
    /* occurrences of each candidate id in the context (the presence / count loops of :59-76, :151-163) */
    for (int64_t t = 0; t < n_context; t++)
        if (context[t] >= 0 && context[t] < vocab) count[context[t]]++;
    /* apply_repetition_penalty (:54-76) */
    if (cfg->repetition_penalty != 1.0f && n_context > 0)
        for (int64_t i = 0; i < vocab; i++)
            if (count[i] > 0) {
                if (c[i].logit < 0.0f) c[i].logit *= cfg->repetition_penalty;
                else c[i].logit /= cfg->repetition_penalty;
            }
    /* apply_frequency_presence_penalty (:143-163) */
    if (!(cfg->frequency_penalty == 0.0f && cfg->presence_penalty == 0.0f) && n_context > 0)
        for (int64_t i = 0; i < vocab; i++)
            if (count[i] > 0) {
                const float freq_loss = (float)count[i] * cfg->frequency_penalty;
                c[i].logit -= (freq_loss + cfg->presence_penalty);
            }
    /* apply_temperature (:79-88) */
    if (cfg->temperature > 0.0f && cfg->temperature != 1.0f) {
        const float inv_temp = 1.0f / cfg->temperature;
        for (int64_t i = 0; i < vocab; i++) c[i].logit *= inv_temp;
    }
    int64_t n = vocab;
    int sorted = 0;
    /* apply_top_k (:107-116) */
    if (cfg->top_k > 0 && cfg->top_k < n) {
        qsort(c, (size_t)n, sizeof(cand_t), cand_cmp);
        sorted = 1;
        n = cfg->top_k;
    }
    /* apply_top_p (:119-147) */
    if (cfg->top_p < 1.0f && n > 1) {
        if (!sorted) qsort(c, (size_t)n, sizeof(cand_t), cand_cmp);
        sorted = 1;
        stage_probs(c, n, probs);
        float cum = 0.0f;
        int64_t cutoff = n - 1;
        for (int64_t i = 0; i < n; i++) {
            cum += probs[i];
            if (cum >= cfg->top_p) {
                cutoff = i;
                break;
            }
        }
        n = cutoff + 1;
    }
    /* apply_min_p (:166-194) */
    if (cfg->min_p > 0.0f && cfg->min_p < 1.0f && n > 1) {
        if (!sorted) qsort(c, (size_t)n, sizeof(cand_t), cand_cmp);
        sorted = 1;
        stage_probs(c, n, probs);
        const float threshold = cfg->min_p * probs[0];
        int64_t kept = 0;
        while (kept < n && probs[kept] >= threshold) kept++;
        if (kept > 0) n = kept;
    }
    for (int64_t i = 0; i < n; i++) {
        ids_out[i] = c[i].id;
        logits_out[i] = c[i].logit;
    }
    free(c);
    free(count);
    free(probs);
    return n;
}

int64_t ao_sample_token_f16(const uint16_t *logits, int64_t vocab, const ao_sampler_config *cfg,
                            const int64_t *context, int64_t n_context, const int64_t *suppress,
                            int64_t n_suppress, uint64_t *rng_state) {
    if (vocab <= 0) return 0;
    /* greedy branch (:241-261) */
    if (cfg->temperature <= 0.0f || cfg->top_k == 1) return ao_greedy_sample_f16(logits, vocab, suppress, n_suppress);
    int64_t *ids = (int64_t *)malloc((size_t)vocab * sizeof(int64_t));
    float *lg = (float *)malloc((size_t)vocab * sizeof(float));
    float *ex = (float *)malloc((size_t)vocab * sizeof(float));
    const int64_t n = ao_sample_candidates_f16(logits, vocab, cfg, context, n_context, suppress, n_suppress, ids, lg);
    int64_t tok = 0;
    if (n > 0) {
        /* final draw (:284-305) */
        float max_l = lg[0];
        for (int64_t i = 1; i < n; i++)
            if (lg[i] > max_l) max_l = lg[i];
        float sum_e = 0.0f;
        for (int64_t i = 0; i < n; i++) {
            ex[i] = exp_f32(lg[i] - max_l);
            sum_e += ex[i];
        }
        if (sum_e <= 0.0f) {
            tok = ids[0];
        } else {
            const float r = ao_rune_rng_next_float32(rng_state) * sum_e;
            float acc = 0.0f;
            tok = ids[n - 1];
            for (int64_t i = 0; i < n; i++) {
                acc += ex[i];
                if (r <= acc) {
                    tok = ids[i];
                    break;
                }
            }
        }
    }
    free(ids);
    free(lg);
    free(ex);
    return tok;
}

/* GGUF block_q8_0: { f16 d; int8 qs[32]; } packed, 34 bytes. */
#define Q8_0_BLOCK_BYTES 34

static inline uint16_t q8_0_weight(const uint8_t *blk, int i) {
    uint16_t d;
    memcpy(&d, blk, 2);
    int8_t q = (int8_t)blk[2 + i];
    return hmul(F2H((float)q), d); /* Scalar[f16](qs[i]) * scale, compute.mojo:1057-1063 */
}

/* dequantize_q8_0, compute.mojo:343-353 */
void ao_dequantize_q8_0(const uint8_t *blocks, uint16_t *out, int64_t n_blocks) {
    for (int64_t b = 0; b < n_blocks; b++)
        for (int i = 0; i < 32; i++) out[b * 32 + i] = q8_0_weight(blocks + b * Q8_0_BLOCK_BYTES, i);
}

/* gemm_q8_0, compute.mojo:1038-1065: per-element f32 products accumulated sequentially. */
int ao_gemm_q8_0(const uint16_t *A, int64_t a_rows, int64_t a_cols, const uint8_t *blocks, int64_t b_rows,
                 uint16_t *C, int64_t c_rows, int64_t c_cols) {
    if (a_rows <= 0 || a_cols <= 0 || b_rows <= 0)
        return ao_fail(AO_ERR_INVALID, "gemm_q8_0: matrix dimensions must be positive");
    if (a_cols % 32 != 0) return ao_fail(AO_ERR_SHAPE, "gemm_q8_0: inner dimension must be a multiple of 32");
    if (c_rows != a_rows || c_cols != b_rows) return ao_fail(AO_ERR_SHAPE, "gemm_q8_0: output matrix shape mismatch");
    const int64_t K = a_cols, bpr = K / 32;
    for (int64_t row = 0; row < a_rows; row++) {
        for (int64_t n = 0; n < b_rows; n++) {
            float sum = 0.0f;
            for (int64_t b = 0; b < bpr; b++) {
                const uint8_t *blk = blocks + (n * bpr + b) * Q8_0_BLOCK_BYTES;
                for (int i = 0; i < 32; i++) sum += H2F(A[row * K + b * 32 + i]) * H2F(q8_0_weight(blk, i));
            }
            C[row * b_rows + n] = F2H(sum);
        }
    }
    return AO_OK;
}

/* ------------------------------------------------------------------ 4-bit and K-quant blocks */

/* GGUF block_q4_0 { f16 d; uint8 qs[16]; } packed, 18 bytes: byte i holds element i in its low
 * nibble and element i + 16 in its high nibble. The reference's BlockQ4_0 (compute.mojo:22-31)
 * names the same two fields in that order. */
#define Q4_0_BLOCK_BYTES 18

/* dequantize_q4_0, compute.mojo:266-280: w = f16((f16(q) - 8) * d). q - 8 is exact in f16, so
 * the single rounding is that of the product (evaluated exactly in f32, rounded once). */
static inline uint16_t q4_0_weight(const uint8_t *blk, int i) {
    uint16_t d;
    memcpy(&d, blk, 2);
    const int q = i < 16 ? (blk[2 + i] & 0x0F) : (blk[2 + i - 16] >> 4);
    return F2H((float)(q - 8) * H2F(d));
}

void ao_dequantize_q4_0(const uint8_t *blocks, uint16_t *out, int64_t n_blocks) {
    for (int64_t b = 0; b < n_blocks; b++)
        for (int i = 0; i < 32; i++) out[b * 32 + i] = q4_0_weight(blocks + b * Q4_0_BLOCK_BYTES, i);
}

/* gemm_q4_0, compute.mojo:876-912: per block, the 16 lower and the 16 upper products are each
 * reduced by the 16-lane reduce_add and added to an f32 sum in that order; C = f16(sum). */
int ao_gemm_q4_0(const uint16_t *A, int64_t a_rows, int64_t a_cols, const uint8_t *blocks, int64_t b_rows,
                 uint16_t *C, int64_t c_rows, int64_t c_cols) {
    if (a_rows <= 0 || a_cols <= 0 || b_rows <= 0)
        return ao_fail(AO_ERR_INVALID, "gemm_q4_0: matrix dimensions must be positive");
    if (a_cols % 32 != 0) return ao_fail(AO_ERR_SHAPE, "gemm_q4_0: inner dimension must be a multiple of 32");
    if (c_rows != a_rows || c_cols != b_rows) return ao_fail(AO_ERR_SHAPE, "gemm_q4_0: output matrix shape mismatch");
    const int64_t K = a_cols, bpr = K / 32;
    uint16_t w[32];
    for (int64_t row = 0; row < a_rows; row++) {
        for (int64_t n = 0; n < b_rows; n++) {
            float sum = 0.0f;
            for (int64_t b = 0; b < bpr; b++) {
                const uint8_t *blk = blocks + (n * bpr + b) * Q4_0_BLOCK_BYTES;
                for (int i = 0; i < 32; i++) w[i] = q4_0_weight(blk, i);
                sum += chunk16_dot_scalar(A + row * K + b * 32, w);
                sum += chunk16_dot_scalar(A + row * K + b * 32 + 16, w + 16);
            }
            C[row * b_rows + n] = F2H(sum);
        }
    }
    return AO_OK;
}

/* GGML's K-quant super-blocks of 256 weights, as GGUF files store them (GGML type 12 = Q4_K and
 * 14 = Q6_K, the ids the reference loader maps at loader/gguf.mojo:20-30). The reference's own
 * BlockQ4_K / BlockQ6_K (compute.mojo:86-100, 183-199) are different, synthetic layouts; these
 * functions restate GGML's published block format (ggml-quants dequantize_row_q4_K /
 * dequantize_row_q6_K, unchanged since GGUF v3) in f32, which is what the library's K-quant
 * GEMVs accumulate against. */
#define Q4_K_BLOCK_BYTES 144
#define Q6_K_BLOCK_BYTES 210

/* 6-bit scale and min of sub-block j (0..7) of a Q4_K super-block. */
static void q4_k_scale_min(const uint8_t *sc, int j, int *scale, int *min) {
    if (j < 4) {
        *scale = sc[j] & 63;
        *min = sc[j + 4] & 63;
    } else {
        *scale = (sc[j + 4] & 0x0F) | ((sc[j - 4] >> 6) << 4);
        *min = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}

/* block_q4_K { f16 d; f16 dmin; uint8 scales[12]; uint8 qs[128]; }: weight 64 g + l (l < 32)
 * is the low nibble of qs[32 g + l] (sub-block 2 g), weight 64 g + 32 + l its high nibble
 * (sub-block 2 g + 1); w = (d * sc) * q - dmin * m in f32 (both products exact, one rounding). */
void ao_dequantize_q4_k(const uint8_t *blocks, float *out, int64_t n_blocks) {
    for (int64_t b = 0; b < n_blocks; b++) {
        const uint8_t *blk = blocks + b * Q4_K_BLOCK_BYTES;
        uint16_t dh, mh;
        memcpy(&dh, blk, 2);
        memcpy(&mh, blk + 2, 2);
        const float d = H2F(dh), dmin = H2F(mh);
        const uint8_t *sc = blk + 4, *qs = blk + 16;
        float *y = out + b * 256;
        for (int g = 0; g < 4; g++) {
            int s0, m0, s1, m1;
            q4_k_scale_min(sc, 2 * g, &s0, &m0);
            q4_k_scale_min(sc, 2 * g + 1, &s1, &m1);
            const float d0 = d * (float)s0, n0 = dmin * (float)m0, d1 = d * (float)s1, n1 = dmin * (float)m1;
            for (int l = 0; l < 32; l++) {
                y[64 * g + l] = d0 * (float)(qs[32 * g + l] & 0x0F) - n0;
                y[64 * g + 32 + l] = d1 * (float)(qs[32 * g + l] >> 4) - n1;
            }
        }
    }
}

/* block_q6_K { uint8 ql[128]; uint8 qh[64]; int8 scales[16]; f16 d; }: for half h (ql + 64 h,
 * qh + 32 h, scales + 8 h) and l < 32, the 6-bit values
 *   q1 = (ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)       -> weight 128 h + l,      scale[l / 16]
 *   q2 = (ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)  -> weight 128 h + l + 32, scale[l / 16 + 2]
 *   q3 = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)       -> weight 128 h + l + 64, scale[l / 16 + 4]
 *   q4 = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)  -> weight 128 h + l + 96, scale[l / 16 + 6]
 * and w = (d * scale) * (q - 32) in f32 (d * scale exact, one rounding). */
void ao_dequantize_q6_k(const uint8_t *blocks, float *out, int64_t n_blocks) {
    for (int64_t b = 0; b < n_blocks; b++) {
        const uint8_t *blk = blocks + b * Q6_K_BLOCK_BYTES;
        uint16_t dh;
        memcpy(&dh, blk + 208, 2);
        const float d = H2F(dh);
        float *y = out + b * 256;
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
            const int8_t *sc = (const int8_t *)(blk + 192 + 8 * h);
            for (int l = 0; l < 32; l++) {
                const int is = l / 16;
                const int q1 = ((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[128 * h + l] = (d * (float)sc[is]) * (float)q1;
                y[128 * h + l + 32] = (d * (float)sc[is + 2]) * (float)q2;
                y[128 * h + l + 64] = (d * (float)sc[is + 4]) * (float)q3;
                y[128 * h + l + 96] = (d * (float)sc[is + 6]) * (float)q4;
            }
        }
    }
}

/* Correctly rounded binary64 -> binary16: round to odd into f32 (24 significant bits, more than
 * the 11 + 2 that f16 needs), then round to nearest even into f16; the sticky odd bit makes the
 * two roundings equal one (Boldo and Melquiond, "When double rounding is odd", 2005). */
static uint16_t ao_f64_to_f16(double x) {
    float f = (float)x;
    if ((double)f != x) {
        if (fabs((double)f) > fabs(x)) f = nextafterf(f, 0.0f); /* toward zero */
        uint32_t b;
        memcpy(&b, &f, 4);
        b |= 1u;
        memcpy(&f, &b, 4);
    }
    return F2H(f);
}

/* The library's f16 K-quant weights (quant.hip): the block's scale products rounded to f16, then
 * one rounding of the weight, in the f16 arithmetic of the reference's dequantize_q4_k_m
 * (compute.mojo:245-262, q * scale + min) and dequantize_q6_k_block (compute.mojo:508-527):
 *   Q4_K  w = f16(a q - b), a = f16(d sc), b = f16(dmin m)   (a fused multiply-add: one rounding)
 *   Q6_K  w = f16(a (q - 32)), a = f16(d sc)
 * d sc and dmin m are exact in f32 (11 x 8 bits), so F2H rounds them once; a q - b is exact in f64
 * (at most 43 significant bits across the f16 exponent range) and ao_f64_to_f16 rounds it once;
 * a (q - 32) is exact in f32. Block fields and weight order as ao_dequantize_q4_k / _q6_k. */
void ao_dequantize_q4_k_f16(const uint8_t *blocks, uint16_t *out, int64_t n_blocks) {
    for (int64_t b = 0; b < n_blocks; b++) {
        const uint8_t *blk = blocks + b * Q4_K_BLOCK_BYTES;
        uint16_t dh, mh;
        memcpy(&dh, blk, 2);
        memcpy(&mh, blk + 2, 2);
        const float d = H2F(dh), dmin = H2F(mh);
        const uint8_t *sc = blk + 4, *qs = blk + 16;
        uint16_t *y = out + b * 256;
        for (int g = 0; g < 4; g++) {
            int s0, m0, s1, m1;
            q4_k_scale_min(sc, 2 * g, &s0, &m0);
            q4_k_scale_min(sc, 2 * g + 1, &s1, &m1);
            const double a0 = H2F(F2H(d * (float)s0)), b0 = H2F(F2H(dmin * (float)m0));
            const double a1 = H2F(F2H(d * (float)s1)), b1 = H2F(F2H(dmin * (float)m1));
            for (int l = 0; l < 32; l++) {
                y[64 * g + l] = ao_f64_to_f16(a0 * (double)(qs[32 * g + l] & 0x0F) - b0);
                y[64 * g + 32 + l] = ao_f64_to_f16(a1 * (double)(qs[32 * g + l] >> 4) - b1);
            }
        }
    }
}

void ao_dequantize_q6_k_f16(const uint8_t *blocks, uint16_t *out, int64_t n_blocks) {
    for (int64_t b = 0; b < n_blocks; b++) {
        const uint8_t *blk = blocks + b * Q6_K_BLOCK_BYTES;
        uint16_t dh;
        memcpy(&dh, blk + 208, 2);
        const float d = H2F(dh);
        uint16_t *y = out + b * 256;
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
            const int8_t *sc = (const int8_t *)(blk + 192 + 8 * h);
            for (int l = 0; l < 32; l++) {
                const int is = l / 16;
                const int q[4] = {((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32,
                                  ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32,
                                  ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32,
                                  ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32};
                for (int j = 0; j < 4; j++) {
                    const float a = H2F(F2H(d * (float)sc[is + 2 * j]));
                    y[128 * h + 32 * j + l] = F2H(a * (float)q[j]);
                }
            }
        }
    }
}

/* ------------------------------------------------------------------ Q4_1, Q5_0, Q5_1 blocks */

/* GGUF block_q4_1 { f16 d; f16 m; uint8 qs[16]; } (20 bytes), block_q5_0 { f16 d; uint8 qh[4];
 * uint8 qs[16]; } (22) and block_q5_1 { f16 d; f16 m; uint8 qh[4]; uint8 qs[16]; } (24), packed.
 * The reference's BlockQ4_1 / BlockQ5_0 / BlockQ5_1 (compute.mojo:35-83) hold the same fields in
 * the same order. Element i < 16 is the low nibble of qs[i], element i + 16 its high nibble; for
 * the 5-bit types bit i % 8 of qh[i / 8] is element i's fifth bit (compute.mojo:309-312). */
#define Q4_1_BLOCK_BYTES 20
#define Q5_0_BLOCK_BYTES 22
#define Q5_1_BLOCK_BYTES 24

static int legacy_block_bytes(int type) { return type == 3 ? Q4_1_BLOCK_BYTES : type == 6 ? Q5_0_BLOCK_BYTES : Q5_1_BLOCK_BYTES; }

/* The 4- or 5-bit value of element i of a block of GGML type 3 (Q4_1), 6 (Q5_0) or 7 (Q5_1). */
static int legacy_q(const uint8_t *blk, int type, int i) {
    const uint8_t *qs = blk + (type == 3 ? 4 : type == 6 ? 6 : 8);
    int q = i < 16 ? (qs[i] & 0x0F) : (qs[i - 16] >> 4);
    if (type != 3) {
        const uint8_t *qh = blk + (type == 6 ? 2 : 4);
        q |= ((qh[i / 8] >> (i % 8)) & 1) << 4;
    }
    return q;
}

/* The reference's f16 weight of element i, every f16 operation rounded once:
 *   Q4_1  w = f16(f16(q * d) + m)         dequantize_q4_1 / gemm_q4_1 (compute.mojo:282-296, 941-942)
 *   Q5_0  w = f16((q + 16 h - 16) * d)    dequantize_q5_0 / gemm_q5_0 (compute.mojo:299-317, 985-986)
 *   Q5_1  w = f16(f16(q5 * d) + m)        dequantize_q5_1 / gemm_q5_1 (compute.mojo:321-340, 1027-1028)
 * q + 16 h - 16 and every f16 conversion of a small integer are exact; q * d is exact in f32
 * (5 x 11 bits) and F2H rounds it once; the sum of two f16 values is exact in f64 (their exponents
 * span at most 41 bits) and ao_f64_to_f16 rounds it once. */
static uint16_t legacy_weight(const uint8_t *blk, int type, int i) {
    uint16_t dh, mh = 0;
    memcpy(&dh, blk, 2);
    if (type != 6) memcpy(&mh, blk + 2, 2);
    const int q = legacy_q(blk, type, i);
    if (type == 6) return F2H((float)(q - 16) * H2F(dh));
    const uint16_t prod = F2H((float)q * H2F(dh));
    return ao_f64_to_f16((double)H2F(prod) + (double)H2F(mh));
}

int ao_dequantize_legacy(int type, const uint8_t *blocks, uint16_t *out, int64_t n_blocks) {
    if (type != 3 && type != 6 && type != 7) return ao_fail(AO_ERR_INVALID, "dequantize: type is not Q4_1, Q5_0 or Q5_1");
    const int bb = legacy_block_bytes(type);
    for (int64_t b = 0; b < n_blocks; b++)
        for (int i = 0; i < 32; i++) out[b * 32 + i] = legacy_weight(blocks + b * bb, type, i);
    return AO_OK;
}

/* gemm_q4_1 (compute.mojo:914-951): per block, the 16 lower and the 16 upper products are each
 * reduced by the 16-lane reduce_add and added to the f32 sum, as gemm_q4_0. gemm_q5_0 / gemm_q5_1
 * (compute.mojo:953-993, 995-1036): per block and i < 16, sum += a_lo * w_lo + a_hi * w_hi (two
 * f32 products, their f32 sum, then the running sum; no contraction). C = f16(sum). */
int ao_gemm_legacy(int type, const uint16_t *A, int64_t a_rows, int64_t a_cols, const uint8_t *blocks, int64_t b_rows,
                   uint16_t *C, int64_t c_rows, int64_t c_cols) {
    if (type != 3 && type != 6 && type != 7) return ao_fail(AO_ERR_INVALID, "gemm: type is not Q4_1, Q5_0 or Q5_1");
    if (a_rows <= 0 || a_cols <= 0 || b_rows <= 0) return ao_fail(AO_ERR_INVALID, "gemm: matrix dimensions must be positive");
    if (a_cols % 32 != 0) return ao_fail(AO_ERR_SHAPE, "gemm: inner dimension must be a multiple of 32");
    if (c_rows != a_rows || c_cols != b_rows) return ao_fail(AO_ERR_SHAPE, "gemm: output matrix shape mismatch");
    const int64_t K = a_cols, bpr = K / 32;
    const int bb = legacy_block_bytes(type);
    uint16_t w[32];
    for (int64_t row = 0; row < a_rows; row++) {
        for (int64_t n = 0; n < b_rows; n++) {
            float sum = 0.0f;
            for (int64_t b = 0; b < bpr; b++) {
                const uint8_t *blk = blocks + (n * bpr + b) * bb;
                const uint16_t *a = A + row * K + b * 32;
                for (int i = 0; i < 32; i++) w[i] = legacy_weight(blk, type, i);
                if (type == 3) {
                    sum += chunk16_dot_scalar(a, w);
                    sum += chunk16_dot_scalar(a + 16, w + 16);
                } else {
                    for (int i = 0; i < 16; i++) {
                        const float lo = H2F(a[i]) * H2F(w[i]), hi = H2F(a[16 + i]) * H2F(w[16 + i]);
                        sum += lo + hi;
                    }
                }
            }
            C[row * b_rows + n] = F2H(sum);
        }
    }
    return AO_OK;
}

/* ------------------------------------------------------------------ Q5_K, Q2_K, Q3_K super-blocks */

/* GGML's other K-quant super-blocks of 256 weights as GGUF files hold them (types 13, 10, 11; the
 * ids of loader/gguf.mojo:26-29). The reference's BlockQ5_K / BlockQ3_K (compute.mojo:131-162) are
 * synthetic layouts and its BlockQ2_K (:164-181) has GGML's fields but dequantize_q2_k_block
 * (:486-504) ignores the scales, so these restate GGML's published format (ggml-quants
 * dequantize_row_q5_K / _q2_K / _q3_K, unchanged since GGUF v3):
 *   block_q5_K { f16 d; f16 dmin; uint8 scales[12]; uint8 qh[32]; uint8 qs[128]; } (176 bytes):
 *     Q4_K's scale packing and nibble order, plus bit 2 g (weight 64 g + l) or 2 g + 1 (weight
 *     64 g + 32 + l) of qh[l] as the fifth bit; w = d sc q - dmin m.
 *   block_q2_K { uint8 scales[16]; uint8 qs[64]; f16 d; f16 dmin; } (84 bytes): for half h, shift
 *     j and l < 32, weight 128 h + 32 j + l is (qs[32 h + l] >> 2 j) & 3, with sub-block
 *     is = 8 h + 2 j + l / 16 whose byte holds the 4-bit scale (low) and min (high);
 *     w = d sc q - dmin m.
 *   block_q3_K { uint8 hmask[32]; uint8 qs[64]; uint8 scales[12]; f16 d; } (110 bytes): the same
 *     2-bit order as Q2_K, minus 4 unless bit 4 h + j of hmask[l] is set, with sixteen 6-bit
 *     scales (low 4 bits: byte j of scales for j < 8, the high nibble of byte j - 8 above; high 2
 *     bits: bits 2 (j / 4) of byte 8 + j % 4), less 32; w = d (sc - 32) q. */
#define Q5_K_BLOCK_BYTES 176
#define Q2_K_BLOCK_BYTES 84
#define Q3_K_BLOCK_BYTES 110

static int q3_k_scale(const uint8_t *sc, int j) {
    const int lo = j < 8 ? (sc[j] & 0x0F) : (sc[j - 8] >> 4);
    const int hi = (sc[8 + j % 4] >> (2 * (j / 4))) & 3;
    return (lo | (hi << 4)) - 32;
}

/* (value, scale-or-a, min-or-b index) of weight i of a block: v is the quantized value as the
 * rule multiplies it, s the sub-block's integer scale, m its integer min (0 for Q3_K). */
static void kquant_fields(int type, const uint8_t *blk, int i, int *v, int *s, int *m, float *d, float *dmin) {
    uint16_t dh = 0, mh = 0;
    if (type == 13) {
        memcpy(&dh, blk, 2);
        memcpy(&mh, blk + 2, 2);
        const uint8_t *qh = blk + 16, *qs = blk + 48;
        const int g = i / 64, l = i % 64, hi = l >= 32, ll = l % 32;
        *v = (hi ? (qs[32 * g + ll] >> 4) : (qs[32 * g + ll] & 0x0F)) | (((qh[ll] >> (2 * g + hi)) & 1) << 4);
        q4_k_scale_min(blk + 4, 2 * g + hi, s, m);
    } else {
        const int h = i / 128, j = (i % 128) / 32, l = i % 32;
        const int is = 8 * h + 2 * j + l / 16;
        if (type == 10) {
            memcpy(&dh, blk + 80, 2);
            memcpy(&mh, blk + 82, 2);
            *v = (blk[16 + 32 * h + l] >> (2 * j)) & 3;
            *s = blk[is] & 0x0F;
            *m = blk[is] >> 4;
        } else {
            memcpy(&dh, blk + 108, 2);
            const int q = (blk[32 + 32 * h + l] >> (2 * j)) & 3;
            *v = q - (((blk[l] >> (4 * h + j)) & 1) ? 0 : 4);
            *s = q3_k_scale(blk + 96, is);
            *m = 0;
        }
    }
    *d = H2F(dh);
    *dmin = H2F(mh);
}

static int kquant_block_bytes(int type) { return type == 13 ? Q5_K_BLOCK_BYTES : type == 10 ? Q2_K_BLOCK_BYTES : Q3_K_BLOCK_BYTES; }

/* GGML's f32 weights: (d sc) q - (dmin m), d sc and dmin m exact in f32, one rounding. */
int ao_dequantize_kquant(int type, const uint8_t *blocks, float *out, int64_t n_blocks) {
    if (type != 10 && type != 11 && type != 13) return ao_fail(AO_ERR_INVALID, "dequantize: type is not Q2_K, Q3_K or Q5_K");
    const int bb = kquant_block_bytes(type);
    for (int64_t b = 0; b < n_blocks; b++)
        for (int i = 0; i < 256; i++) {
            int v, sc, m;
            float d, dmin;
            kquant_fields(type, blocks + b * bb, i, &v, &sc, &m, &d, &dmin);
            out[b * 256 + i] = (d * (float)sc) * (float)v - dmin * (float)m;
        }
    return AO_OK;
}

/* The library's f16 weights, the form of the Q4_K / Q6_K rules: a = f16(d sc), b = f16(dmin m),
 * w = f16(a q - b) with one rounding (Q5_K, Q2_K), w = f16(a q) (Q3_K). */
int ao_dequantize_kquant_f16(int type, const uint8_t *blocks, uint16_t *out, int64_t n_blocks) {
    if (type != 10 && type != 11 && type != 13) return ao_fail(AO_ERR_INVALID, "dequantize: type is not Q2_K, Q3_K or Q5_K");
    const int bb = kquant_block_bytes(type);
    for (int64_t b = 0; b < n_blocks; b++)
        for (int i = 0; i < 256; i++) {
            int v, sc, m;
            float d, dmin;
            kquant_fields(type, blocks + b * bb, i, &v, &sc, &m, &d, &dmin);
            const double a = H2F(F2H(d * (float)sc)), bm = H2F(F2H(dmin * (float)m));
            out[b * 256 + i] = ao_f64_to_f16(a * (double)v - bm);
        }
    return AO_OK;
}

/* ------------------------------------------------------------------ KV cache */

/* KVCache.append, mimir_well.mojo:488-501 */
int ao_kv_append(ao_kv *kv, int64_t layer, int64_t pos, const uint16_t *key, int64_t key_size,
                 const uint16_t *val, int64_t val_size) {
    if (layer < 0 || layer >= kv->num_layers) return ao_fail(AO_ERR_INVALID, "KVCache.append: layer_idx out of bounds");
    if (pos < 0) return ao_fail(AO_ERR_INVALID, "KVCache.append: pos must be non-negative");
    if (key_size < kv->kv_dim || val_size < kv->kv_dim) return ao_fail(AO_ERR_SHAPE, "KVCache.append: key/val width mismatch");
    int64_t slot = pos % kv->max_seq;
    int64_t off = (layer * kv->max_seq + slot) * kv->kv_dim;
    memcpy(kv->k + off, key, (size_t)kv->kv_dim * 2);
    memcpy(kv->v + off, val, (size_t)kv->kv_dim * 2);
    return AO_OK;
}

/* KVCache.get_k_slice / get_v_slice, mimir_well.mojo:503-521 */
int ao_kv_slice(const ao_kv *kv, int64_t layer, int64_t seq_len, const uint16_t **k_out, const uint16_t **v_out) {
    if (layer < 0 || layer >= kv->num_layers) return ao_fail(AO_ERR_INVALID, "KVCache.get_k_slice: layer_idx out of bounds");
    if (seq_len <= 0 || seq_len > kv->max_seq) return ao_fail(AO_ERR_INVALID, "KVCache.get_k_slice: seq_len out of bounds");
    int64_t off = layer * kv->max_seq * kv->kv_dim;
    *k_out = kv->k + off;
    *v_out = kv->v + off;
    return AO_OK;
}

/* ------------------------------------------------------------------ forward pass */

int64_t ao_forward_scratch_elems(const ao_config *c) {
    int64_t kvd = (c->dim / c->n_heads) * c->n_kv_heads;
    /* x, residual, q, k, v, attn_out, up, gate, logits (inference.mojo:166-259, 458-503) */
    return 4 * c->dim + 2 * kvd + 2 * c->ffn + c->vocab + 64;
}

/* TransformerBlock.forward single-device path, inference.mojo:162-275. */
static int block_forward(const ao_model *m, int64_t l, uint16_t *x, ao_kv *kv, int64_t start_pos, uint16_t *ws) {
    const ao_config *c = &m->cfg;
    const int64_t dim = c->dim, hd = dim / c->n_heads, kvd = hd * c->n_kv_heads, ffn = c->ffn;
    uint16_t *residual = ws;
    uint16_t *q = residual + dim;
    uint16_t *k = q + dim;
    uint16_t *v = k + kvd;
    uint16_t *attn = v + kvd;
    uint16_t *up = attn + dim;
    uint16_t *gate = up + ffn;
    int rc;
    memcpy(residual, x, (size_t)dim * 2);                                  /* :166-169 */
    if ((rc = ao_rmsnorm_f16(x, 1, dim, m->attn_norm[l], dim, c->eps))) return rc; /* :171 */
    if ((rc = ao_gemm_f16(x, 1, dim, m->wq[l], dim, dim, q, 1, dim))) return rc;   /* :194-196 */
    if ((rc = ao_gemm_f16(x, 1, dim, m->wk[l], kvd, dim, k, 1, kvd))) return rc;
    if ((rc = ao_gemm_f16(x, 1, dim, m->wv[l], kvd, dim, v, 1, kvd))) return rc;
    if ((rc = ao_rope_f16(q, 1, dim, k, 1, kvd, start_pos, hd, c->theta))) return rc; /* :200 */
    if ((rc = ao_kv_append(kv, l, start_pos, k, kvd, v, kvd))) return rc;            /* :203 */
    int64_t active = start_pos + 1 < kv->max_seq ? start_pos + 1 : kv->max_seq;     /* :204 */
    const uint16_t *ks, *vs;
    if ((rc = ao_kv_slice(kv, l, active, &ks, &vs))) return rc;
    ao_attn_gqa(q, 1, ks, kvd, vs, kvd, attn, 1, active, hd, c->n_heads, c->n_kv_heads); /* :210-219 */
    if ((rc = ao_gemm_f16(attn, 1, dim, m->wo[l], dim, dim, x, 1, dim))) return rc;    /* :227 */
    ao_residual_add_f16(x, residual, dim);                                             /* :231-232 */
    memcpy(residual, x, (size_t)dim * 2);                                              /* :235-236 */
    if ((rc = ao_rmsnorm_f16(x, 1, dim, m->ffn_norm[l], dim, c->eps))) return rc;     /* :238 */
    if ((rc = ao_gemm_f16(x, 1, dim, m->w_up[l], ffn, dim, up, 1, ffn))) return rc;   /* :254-255 */
    if ((rc = ao_gemm_f16(x, 1, dim, m->w_gate[l], ffn, dim, gate, 1, ffn))) return rc;
    ao_silu_f16(gate, ffn);                                                            /* :258 */
    ao_mul_f16(up, gate, ffn);                                                         /* :259-260 */
    if ((rc = ao_gemm_f16(up, 1, ffn, m->w_down[l], dim, ffn, x, 1, dim))) return rc; /* :268 */
    ao_residual_add_f16(x, residual, dim);                                             /* :272-273 */
    return AO_OK;
}

/* forward_pass, inference.mojo:424-518. */
int ao_forward_partial(const ao_model *m, ao_kv *kv, const int64_t *tokens, int64_t n_tokens, int64_t start_pos,
                       int64_t n_layers_run, uint16_t *scratch, uint16_t *logits_out, int64_t *next_token) {
    const ao_config *c = &m->cfg;
    if (n_tokens == 0) { /* :446-447 */
        *next_token = 0;
        return AO_OK;
    }
    int64_t idx = start_pos < 0 ? 0 : start_pos; /* :449-450 */
    if (idx > n_tokens - 1) idx = n_tokens - 1;
    int64_t tok = tokens[idx];
    if (tok < 0 || tok >= c->vocab) return ao_fail(AO_ERR_INVALID, "Prompt token ID is outside the embedding vocabulary");
    uint16_t *x = scratch;
    uint16_t *ws = x + c->dim;
    memcpy(x, m->token_embd + tok * c->dim, (size_t)c->dim * 2); /* :461-467 */
    int rc;
    for (int64_t l = 0; l < n_layers_run; l++)
        if ((rc = block_forward(m, l, x, kv, start_pos, ws))) return rc;
    float eps = c->eps > 0.0f ? c->eps : 1e-5f; /* :484-488 */
    if ((rc = ao_rmsnorm_f16(x, 1, c->dim, m->output_norm, c->dim, eps))) return rc;
    uint16_t *logits = ws; /* the per-layer workspace is released by then (:275) */
    if ((rc = ao_gemm_f16(x, 1, c->dim, m->output, c->vocab, c->dim, logits, 1, c->vocab))) return rc; /* :495-505 */
    if (logits_out) memcpy(logits_out, logits, (size_t)c->vocab * 2);
    *next_token = ao_argmax_f16(logits, c->vocab); /* :508-515 */
    return AO_OK;
}

int ao_forward_pass(const ao_model *m, ao_kv *kv, const int64_t *tokens, int64_t n_tokens, int64_t start_pos,
                    uint16_t *scratch, uint16_t *logits_out, int64_t *next_token) {
    return ao_forward_partial(m, kv, tokens, n_tokens, start_pos, m->cfg.n_layers, scratch, logits_out, next_token);
}

/* generation_stop_reason, aesir.mojo:195-212. Returns -1 to continue. */
int ao_generation_stop_reason(int64_t token, int64_t eos, int64_t generated_count, int64_t max_new,
                              const int64_t *stop_tokens, int64_t n_stop, int64_t next_position, int64_t ctx_len) {
    if (eos >= 0 && token == eos) return 0;
    for (int64_t i = 0; i < n_stop; i++)
        if (stop_tokens[i] == token) return 1;
    if (generated_count >= max_new) return 2;
    if (next_position >= ctx_len) return 3;
    return -1;
}

/* AesirEngine._run_generation, aesir.mojo:323-462 (token IDs in and out; no text side). */
int ao_generate(const ao_model *m, ao_kv *kv, const int64_t *prompt, int64_t n_prompt, int64_t max_new, int64_t eos,
                const int64_t *stop_tokens, int64_t n_stop, uint16_t *scratch, int64_t *out_tokens, int64_t *n_out,
                int32_t *stop_reason, uint16_t *last_logits) {
    const int64_t ctx_len = m->cfg.ctx_len;
    *n_out = 0;
    if (max_new <= 0) return ao_fail(AO_ERR_INVALID, "GenerationConfig max_new_tokens must be a positive integer");
    if (max_new > ctx_len) return ao_fail(AO_ERR_INVALID, "GenerationConfig max_new_tokens exceeds context_length boundary");
    if (n_prompt <= 0) return ao_fail(AO_ERR_INVALID, "RuneWeaver produced no prompt tokens");
    if (n_prompt > ctx_len) return ao_fail(AO_ERR_INVALID, "Prompt token count exceeds the model context length");
    int64_t *current = (int64_t *)malloc(sizeof(int64_t) * (size_t)(n_prompt + max_new + 1));
    if (!current) return ao_fail(AO_ERR_EXHAUSTED, "oracle: host allocation failed");
    memcpy(current, prompt, sizeof(int64_t) * (size_t)n_prompt);
    int64_t n_cur = n_prompt, next = 0;
    int rc = AO_OK;
    for (int64_t p = 0; p < n_prompt; p++) /* prefill by position, :358-374 */
        if ((rc = ao_forward_pass(m, kv, current, n_cur, p, scratch, last_logits, &next))) goto done;
    int reason = -1;
    for (int64_t it = 0; it < max_new; it++) { /* :381-445 */
        out_tokens[(*n_out)++] = next;
        current[n_cur++] = next;
        if (next == eos) {
            reason = 0;
            break;
        }
        int is_stop = 0;
        for (int64_t s = 0; s < n_stop; s++) is_stop |= stop_tokens[s] == next;
        if (is_stop) {
            reason = 1;
            break;
        }
        int64_t next_position = n_cur - 1;
        reason = ao_generation_stop_reason(next, eos, *n_out, max_new, stop_tokens, n_stop, next_position, ctx_len);
        if (reason >= 0) break;
        if ((rc = ao_forward_pass(m, kv, current, n_cur, next_position, scratch, last_logits, &next))) goto done;
    }
    if (reason < 0) reason = 2;
    *stop_reason = reason;
done:
    free(current);
    return rc;
}

/* ------------------------------------------------------------------ synthetic inputs */

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* RuneRNG.next_u64, sampler.mojo:34-37: the state itself is advanced through the mixer. */
uint64_t ao_rune_rng_next(uint64_t *state) {
    uint64_t s = *state;
    s = (s ^ (s >> 30)) * 0xBF58476D1CE4E5B9ULL;
    s = (s ^ (s >> 27)) * 0x94D049BB133111EBULL;
    *state = s;
    return s ^ (s >> 31);
}

#define GOLDEN 0x9E3779B97F4A7C15ULL

/* Counter-based normal: element i of (seed, stream) from two mixer outputs, Box-Muller in f64.
 * The same formula runs on the device for weights too large to generate on the host. */
static double normal_at(uint64_t base, int64_t i) {
    uint64_t a = mix64(base + (uint64_t)(2 * i + 1) * GOLDEN);
    uint64_t b = mix64(base + (uint64_t)(2 * i + 2) * GOLDEN);
    double u1 = (double)((a >> 40) + 1) * (1.0 / 16777216.0); /* (0, 1] */
    double u2 = (double)(b >> 40) * (1.0 / 16777216.0);       /* [0, 1) */
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void ao_fill_normal_f32(float *dst, int64_t n, uint64_t seed, uint64_t stream, float mean, float std) {
    uint64_t base = mix64(seed ^ mix64(stream + GOLDEN));
    for (int64_t i = 0; i < n; i++) dst[i] = (float)((double)mean + (double)std * normal_at(base, i));
}

void ao_fill_normal_f16(uint16_t *dst, int64_t n, uint64_t seed, uint64_t stream, float mean, float std) {
    uint64_t base = mix64(seed ^ mix64(stream + GOLDEN));
    for (int64_t i = 0; i < n; i++) dst[i] = F2H((float)((double)mean + (double)std * normal_at(base, i)));
}
