// The full sampler stack on the device: sample_token_from_logits (core/sampler.mojo:217-305).
//
//   prepare   one thread per vocabulary entry: sanitize_logit (:9-14), the suppress mask (:197-211),
//             the repetition and frequency / presence penalties (:54-76, :143-163) from a context
//             histogram built with integer atomics (order-independent, so deterministic), and the
//             temperature scale (:79-88); f32 arithmetic in the reference's order
//   sort      when top-k, top-p or min-p truncates: one stable LSD radix sort (rocPRIM) of
//             (descending logit key, index). Equal logits (-0 == +0) keep index order, which is the
//             order the reference's stable insertion sort (:92-104) produces; every later stage of
//             the stack sees an already sorted prefix, so one sort serves all of them
//   tail      one workgroup: the f32 running sums of apply_top_p, apply_min_p and the final draw
//             in one lane in candidate order (f32 addition is not associative; the sums must follow
//             the reference's order to choose the same token), with the next LDS tile of exps
//             computed by the other waves meanwhile. The draw's inverse-CDF walk repeats the sum's
//             running values, so the sum records one every 32 terms and the walk re-adds one block
//   greedy    temperature <= 0 or top_k == 1: the first maximum of the sanitized, masked logits
//
// The random number comes from RuneRNG on the host (one draw per sampled token, consumed only
// when the reference consumes it: a positive final sum). exp is evaluated as the correctly
// rounded f32 value (f64 exp rounded once) so that the CPU oracle computes the same bits.
#include <cstring>
#include <rocprim/device/device_radix_sort.hpp>

#include "common.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aesir {

constexpr int kSThreads = 256;
constexpr int kTailThreads = 256;

__device__ __forceinline__ float sanitize_logit(float v) { return (isnan(v) || isinf(v)) ? -1e9f : v; }
__device__ __forceinline__ float exp_f32(float x) { return (float)exp((double)x); }

// Radix key whose ascending order is descending logit order (-0 folded onto +0).
__device__ __forceinline__ uint32_t desc_key(float v) {
    if (v == 0.0f) v = 0.0f;
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const uint32_t asc = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ~asc;
}

struct SampleParams {
    float repetition_penalty, frequency_penalty, presence_penalty, inv_temp;
    int apply_rep, apply_freq, apply_temp, sort;
    int64_t top_k;  // > 0: truncate to top_k after the sort
    float top_p;    // < 1: nucleus
    float min_p;    // in (0, 1): min-p
    float u;        // RuneRNG.next_float32 for the draw
};

__global__ void sampler_clear_kernel(int32_t *__restrict__ counts, uint8_t *__restrict__ mask, int64_t V) {
    for (int64_t i = (int64_t)blockIdx.x * kSThreads + threadIdx.x; i < V; i += (int64_t)gridDim.x * kSThreads) {
        counts[i] = 0;
        mask[i] = 0;
    }
}

// Occurrence counts of the context tokens and the suppress flags (ids outside the vocabulary
// never match a candidate in the reference, so they are skipped).
__global__ void sampler_mark_kernel(const int64_t *__restrict__ ctx, int64_t n_ctx, const int64_t *__restrict__ sup,
                                    int64_t n_sup, int32_t *__restrict__ counts, uint8_t *__restrict__ mask,
                                    int64_t V) {
    for (int64_t i = (int64_t)blockIdx.x * kSThreads + threadIdx.x; i < n_ctx + n_sup;
         i += (int64_t)gridDim.x * kSThreads) {
        if (i < n_ctx) {
            const int64_t t = ctx[i];
            if (t >= 0 && t < V) atomicAdd(&counts[t], 1);
        } else {
            const int64_t t = sup[i - n_ctx];
            if (t >= 0 && t < V) mask[t] = 1;
        }
    }
}

__global__ void sampler_prepare_kernel(const h16 *__restrict__ logits, int64_t V, const int32_t *__restrict__ counts,
                                       const uint8_t *__restrict__ mask, SampleParams p, float *__restrict__ vals,
                                       uint32_t *__restrict__ keys, int32_t *__restrict__ idx) {
    for (int64_t i = (int64_t)blockIdx.x * kSThreads + threadIdx.x; i < V; i += (int64_t)gridDim.x * kSThreads) {
        float v = sanitize_logit((float)logits[i]);
        if (mask[i]) v = -1e9f;
        const int32_t c = counts[i];
        if (p.apply_rep && c > 0) v = v < 0.0f ? v * p.repetition_penalty : v / p.repetition_penalty;
        if (p.apply_freq && c > 0) {
            const float freq_loss = (float)c * p.frequency_penalty;
            v -= (freq_loss + p.presence_penalty);
        }
        if (p.apply_temp) v *= p.inv_temp;
        vals[i] = v;
        if (p.sort) {
            keys[i] = desc_key(v);
            idx[i] = (int32_t)i;
        }
    }
}

// Greedy branch (:241-261): best = 0, max = value of index 0, strict '>' ascending; values are
// sanitized and suppressed ones are -1e9. Equivalent to the lowest index of the maximum.
__global__ __launch_bounds__(1024) void sampler_greedy_kernel(const h16 *__restrict__ logits, int64_t V,
                                                              const uint8_t *__restrict__ mask, int64_t *out) {
    __shared__ float bv[1024];
    __shared__ int64_t bi[1024];
    const int tid = threadIdx.x;
    float best = -INFINITY;
    int64_t besti = -1;
    // strided (coalesced) scan; each thread sees its indices in increasing order, so strict '>'
    // keeps its first maximum, and the tree below resolves equal values to the lower index
    for (int64_t i = tid; i < V; i += 1024) {
        float v = sanitize_logit((float)logits[i]);
        if (mask && mask[i]) v = -1e9f;
        if (besti < 0 || v > best) {
            best = v;
            besti = i;
        }
    }
    bv[tid] = best;
    bi[tid] = besti;
    __syncthreads();
    for (int st = 512; st > 0; st >>= 1) {
        if (tid < st) {
            // the larger value wins; equal values go to the lower index (first maximum)
            const bool take = bi[tid + st] >= 0 &&
                              (bi[tid] < 0 || bv[tid + st] > bv[tid] || (bv[tid + st] == bv[tid] && bi[tid + st] < bi[tid]));
            if (take) {
                bv[tid] = bv[tid + st];
                bi[tid] = bi[tid + st];
            }
        }
        __syncthreads();
    }
    if (tid == 0) {
        out[0] = bi[0] < 0 ? 0 : bi[0];
        out[1] = 0;  // no random number consumed
    }
}

// Truncations and the draw over the candidate list: value i is vals[order ? order[i] : i].
// Every running f32 sum of the reference is evaluated in candidate order by lane 0 of wave 0
// (f32 addition is not associative, so the order fixes the token drawn). The terms come from
// two LDS tiles: while lane 0 adds one tile, waves 1-3 compute the next tile's terms into the
// other, so the exps cost nothing beside the serial adds.
constexpr int kSeqTile = 4096;   // terms per LDS tile (two tiles)
constexpr int kMarkBlock = 32;   // terms per recorded running sum of the final draw's sum

// Lane 0's adds over one tile, acc += buf[e] for e in [0, cnt), 32 terms per block with the next
// block's LDS reads in flight. kHit: stops at the first e with target <= acc (returned in hit,
// -1 when none); a block is added first and re-added term by term only when the target falls
// inside it (terms are >= 0, so acc never decreases). kMarks: marks[b] = acc after block b.
template <bool kHit, bool kMarks>
__device__ __forceinline__ float chain_tile(const float *buf, int cnt, float acc, float target, int &hit,
                                            float *marks) {
    const int nb = cnt / kMarkBlock;
    f32x4 ra[8], rb[8];
    auto load = [&](f32x4(&r)[8], int b) {
#pragma unroll
        for (int q = 0; q < 8; q++) r[q] = *reinterpret_cast<const f32x4 *>(&buf[kMarkBlock * b + 4 * q]);
    };
    auto add = [&](const f32x4(&r)[8], int b) -> bool {
        float a = acc;
#pragma unroll
        for (int q = 0; q < 8; q++)
#pragma unroll
            for (int u = 0; u < 4; u++) a += r[q][u];
        if (kHit && target <= a) {
            float c = acc;
#pragma unroll
            for (int q = 0; q < 8; q++)
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    c += r[q][u];
                    if (target <= c) {
                        hit = kMarkBlock * b + 4 * q + u;
                        acc = c;
                        return true;
                    }
                }
        }
        acc = a;
        if (kMarks) marks[b] = a;
        return false;
    };
    hit = -1;
    if (nb > 0) load(ra, 0);
    for (int b = 0; b < nb; b += 2) {
        if (b + 1 < nb) load(rb, b + 1);
        if (add(ra, b)) return acc;
        if (b + 1 < nb) {
            if (b + 2 < nb) load(ra, b + 2);
            if (add(rb, b + 1)) return acc;
        }
    }
    for (int e = kMarkBlock * nb; e < cnt; e++) {  // the short last block of the last tile
        acc += buf[e];
        if (kHit && target <= acc) {
            hit = e;
            return acc;
        }
    }
    if (kMarks && cnt % kMarkBlock) marks[nb] = acc;
    return acc;
}

// acc_i = acc_{i-1} + term(i) in f32 over i in [0, m), m >= 1, in index order. Returns the first
// i with target <= acc_i (m when none) under kHit, else m; the running sum where the chain
// stopped goes to total (every thread). kMarks: marks[j] = acc at the end of term block j.
// Enter and leave with the workgroup converged; tile0/tile1 and n_sh/f_sh are free on entry.
template <bool kHit, bool kMarks, class Term>
__device__ __forceinline__ int64_t ordered_chain(float *tile0, float *tile1, int64_t m, Term term, float target,
                                                 float *marks, float &total, int64_t *n_sh, float *f_sh) {
    const int tid = threadIdx.x;
    const int64_t nt = (m + kSeqTile - 1) / kSeqTile;
    auto tile_cnt = [&](int64_t k) -> int {
        const int64_t r = m - k * kSeqTile;
        return (int)(r < kSeqTile ? r : kSeqTile);
    };
    {
        const int c = tile_cnt(0);
        for (int e = tid; e < c; e += kTailThreads) tile0[e] = term((int64_t)e);
    }
    __syncthreads();
    float acc = 0.0f;
    int64_t hit = m;
    for (int64_t k = 0; k < nt; k++) {
        float *cur = (k & 1) ? tile1 : tile0;
        float *nxt = (k & 1) ? tile0 : tile1;
        if (tid < 64) {
            if (tid == 0) {
                int he;
                acc = chain_tile<kHit, kMarks>(cur, tile_cnt(k), acc, target, he,
                                               kMarks ? marks + k * (kSeqTile / kMarkBlock) : nullptr);
                // two slots: the others read slot k&1 between barriers k and k+1, lane 0 writes
                // slot (k+1)&1 only after barrier k
                if (kHit) n_sh[k & 1] = he >= 0 ? k * kSeqTile + he : m;
            }
        } else if (k + 1 < nt) {
            const int64_t base = (k + 1) * kSeqTile;
            const int c = tile_cnt(k + 1);
            for (int e = tid - 64; e < c; e += kTailThreads - 64) nxt[e] = term(base + e);
        }
        __syncthreads();
        if (kHit) {
            hit = n_sh[k & 1];
            if (hit < m) break;
        }
    }
    if (tid == 0) *f_sh = acc;
    __syncthreads();
    total = *f_sh;
    __syncthreads();
    return hit;
}

__global__ __launch_bounds__(kTailThreads) void sampler_tail_kernel(const float *__restrict__ vals,
                                                                    const int32_t *__restrict__ order, int64_t V,
                                                                    SampleParams p, float *__restrict__ marks,
                                                                    int64_t *out) {
    __shared__ __align__(16) float tile[2][kSeqTile];
    __shared__ float red[kTailThreads];
    __shared__ int64_t ired[kTailThreads];
    __shared__ int64_t n_sh[2];
    __shared__ float f_sh;
    const int tid = threadIdx.x;
    auto val = [&](int64_t i) -> float { return vals[order ? order[i] : i]; };
    int64_t n = V;
    if (p.top_k > 0 && p.top_k < n) n = p.top_k;  // apply_top_k (:107-116)

    if (p.top_p < 1.0f && n > 1) {  // apply_top_p (:119-147): exps relative to the first (largest) logit
        const float mx = val(0);
        float sum, stop;
        ordered_chain<false, false>(tile[0], tile[1], n, [&](int64_t i) { return exp_f32(val(i) - mx); }, 0.0f,
                                    nullptr, sum, n_sh, &f_sh);
        const int64_t cut = ordered_chain<true, false>(
            tile[0], tile[1], n,
            [&](int64_t i) {
                const float e = exp_f32(val(i) - mx);
                return sum > 0.0f ? e / sum : e;
            },
            p.top_p, nullptr, stop, n_sh, &f_sh);
        n = cut < n ? cut + 1 : n;
    }
    if (p.min_p > 0.0f && p.min_p < 1.0f && n > 1) {  // apply_min_p (:166-194)
        const float mx = val(0);
        float sum;
        ordered_chain<false, false>(tile[0], tile[1], n, [&](int64_t i) { return exp_f32(val(i) - mx); }, 0.0f,
                                    nullptr, sum, n_sh, &f_sh);
        const float e0 = exp_f32(0.0f);  // the first candidate's exp (val(0) - mx = 0)
        const float p0 = sum > 0.0f ? e0 / sum : e0;
        const float threshold = p.min_p * p0;
        // kept = the first index whose probability falls below the threshold (each test is
        // independent of the others, so the tile is searched in parallel)
        int64_t kept = n;
        for (int64_t t0 = 0; t0 < n && kept == n; t0 += kSeqTile) {
            const int cnt = (int)(n - t0 < kSeqTile ? n - t0 : kSeqTile);
            for (int e = tid; e < cnt; e += kTailThreads) tile[0][e] = exp_f32(val(t0 + e) - mx);
            __syncthreads();
            int first = cnt;
            for (int e = tid; e < cnt; e += kTailThreads) {
                const float pr = sum > 0.0f ? tile[0][e] / sum : tile[0][e];
                if (!(pr >= threshold)) {
                    first = e;
                    break;
                }
            }
            red[tid] = (float)first;  // exact: indices < 2^24
            __syncthreads();
            for (int st = kTailThreads / 2; st > 0; st >>= 1) {
                if (tid < st) red[tid] = fminf(red[tid], red[tid + st]);
                __syncthreads();
            }
            if ((int)red[0] < cnt) kept = t0 + (int)red[0];
            __syncthreads();
        }
        n = kept > 0 ? kept : n;
    }

    // final draw (:284-305): max over the candidates, exps, sequential sum, inverse CDF
    float mx = -INFINITY;
    for (int64_t i = tid; i < n; i += kTailThreads) mx = fmaxf(mx, val(i));
    red[tid] = mx;
    __syncthreads();
    for (int st = kTailThreads / 2; st > 0; st >>= 1) {
        if (tid < st) red[tid] = fmaxf(red[tid], red[tid + st]);
        __syncthreads();
    }
    mx = red[0];
    __syncthreads();
    float sum_e;
    ordered_chain<false, true>(tile[0], tile[1], n, [&](int64_t i) { return exp_f32(val(i) - mx); }, 0.0f, marks,
                               sum_e, n_sh, &f_sh);
    const int64_t first = order ? order[0] : 0;
    if (!(sum_e > 0.0f)) {
        if (tid == 0) {
            out[0] = first;
            out[1] = 0;
        }
        return;
    }
    // The draw's running sum is the sum pass's running sum term for term (same terms, same order),
    // so the first i with r <= acc_i lies in the first block whose recorded end sum reaches r;
    // blocks ending below r form a prefix (acc never decreases) and are counted in parallel, and
    // that block is re-added from the previous block's recorded sum.
    const float r = p.u * sum_e;
    const int64_t nb = (n + kMarkBlock - 1) / kMarkBlock;
    int64_t below = 0;
    for (int64_t j = tid; j < nb; j += kTailThreads) below += marks[j] < r ? 1 : 0;
    ired[tid] = below;
    __syncthreads();
    for (int st = kTailThreads / 2; st > 0; st >>= 1) {
        if (tid < st) ired[tid] += ired[tid + st];
        __syncthreads();
    }
    const int64_t jb = ired[0];
    int64_t pick = n - 1;
    if (jb < nb) {
        const int64_t i0 = jb * kMarkBlock;
        const int c = (int)(n - i0 < kMarkBlock ? n - i0 : kMarkBlock);
        if (tid < c) tile[0][tid] = exp_f32(val(i0 + tid) - mx);
        __syncthreads();
        if (tid == 0) {
            float acc = jb > 0 ? marks[jb - 1] : 0.0f;
            for (int e = 0; e < c; e++) {
                acc += tile[0][e];
                if (r <= acc) {
                    pick = i0 + e;
                    break;
                }
            }
        }
    }
    if (tid == 0) {
        out[0] = order ? order[pick] : pick;
        out[1] = 1;
    }
}

// Device workspace of the sampler, grown on demand (never inside a captured graph).
struct SamplerWork {
    int64_t cap_v = 0, cap_ctx = 0;
    int32_t *counts = nullptr;
    uint8_t *mask = nullptr;
    float *vals = nullptr;
    uint32_t *keys = nullptr, *keys_out = nullptr;
    int32_t *idx = nullptr, *idx_out = nullptr;
    float *marks = nullptr;    // the final draw's running sum at the end of every kMarkBlock terms
    int64_t *lists = nullptr;  // context tokens then suppress ids
    int64_t *result = nullptr;
    void *sort_tmp = nullptr;
    size_t sort_tmp_bytes = 0;
};

static void free_work(SamplerWork *w) {
    void *ps[] = {w->counts, w->mask, w->vals, w->keys, w->keys_out, w->idx, w->idx_out, w->marks,
                  w->lists, w->result, w->sort_tmp};
    for (void *p : ps)
        if (p) (void)hipFree(p);
    *w = SamplerWork{};
}

void sampler_release(aesir_ctx *ctx) {
    if (!ctx->sampler) return;
    free_work(ctx->sampler);
    delete ctx->sampler;
    ctx->sampler = nullptr;
}

static int32_t ensure_work(aesir_ctx *ctx, int64_t V, int64_t n_lists) {
    if (!ctx->sampler) ctx->sampler = new SamplerWork();
    SamplerWork *w = ctx->sampler;
    if (V > w->cap_v) {
        AESIR_HIP_TRY(hipStreamSynchronize(ctx->stream));
        const int64_t keep_lists = w->cap_ctx;
        int64_t *old_lists = w->lists, *old_result = w->result;
        w->lists = nullptr;
        w->result = nullptr;
        free_work(w);
        w->lists = old_lists;
        w->result = old_result;
        w->cap_ctx = keep_lists;
        AESIR_HIP_TRY(hipMalloc((void **)&w->counts, (size_t)V * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->mask, (size_t)V));
        AESIR_HIP_TRY(hipMalloc((void **)&w->vals, (size_t)V * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->keys, (size_t)V * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->keys_out, (size_t)V * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->idx, (size_t)V * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->idx_out, (size_t)V * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->marks, (size_t)(V / kMarkBlock + 1) * 4));
        size_t bytes = 0;
        AESIR_HIP_TRY(rocprim::radix_sort_pairs(nullptr, bytes, w->keys, w->keys_out, w->idx, w->idx_out,
                                                (unsigned)V, 0, 32, ctx->stream));
        AESIR_HIP_TRY(hipMalloc(&w->sort_tmp, bytes));
        w->sort_tmp_bytes = bytes;
        w->cap_v = V;
    }
    if (n_lists > w->cap_ctx || !w->lists) {
        AESIR_HIP_TRY(hipStreamSynchronize(ctx->stream));
        if (w->lists) (void)hipFree(w->lists);
        w->lists = nullptr;
        const int64_t cap = n_lists > 1024 ? n_lists : 1024;
        AESIR_HIP_TRY(hipMalloc((void **)&w->lists, (size_t)cap * 8));
        w->cap_ctx = cap;
    }
    if (!w->result) AESIR_HIP_TRY(hipMalloc((void **)&w->result, 16));
    return AESIR_OK;
}

// RuneRNG.next_u64 / next_float32 (core/sampler.mojo:34-42).
static uint64_t rune_next(uint64_t *state) {
    uint64_t s = *state;
    s = (s ^ (s >> 30)) * 0xBF58476D1CE4E5B9ULL;
    s = (s ^ (s >> 27)) * 0x94D049BB133111EBULL;
    *state = s;
    return s ^ (s >> 31);
}

}  // namespace aesir

using namespace aesir;

extern "C" {

uint64_t aesir_rune_rng_next(uint64_t *state) { return state ? rune_next(state) : 0; }

int32_t aesir_sample_token(aesir_ctx *ctx, const void *logits, int64_t vocab, const aesir_sampler_config *cfg,
                           const int64_t *context, int64_t n_context, const int64_t *suppress, int64_t n_suppress,
                           uint64_t *rng_state, int64_t *token) {
    AESIR_TRY(bind(ctx));
    if (!cfg || !rng_state || !token) return fail(AESIR_ERR_INVALID, "sample_token: null argument");
    if (vocab <= 0) {  // sampler.mojo:232-233
        *token = 0;
        return AESIR_OK;
    }
    if (!logits) return fail(AESIR_ERR_INVALID, "sample_token: null logits");
    if (vocab > 2147483647) return fail(AESIR_ERR_UNSUPPORTED, "sample_token: more than 2^31-1 logits");
    if (n_context < 0 || n_suppress < 0 || (n_context > 0 && !context) || (n_suppress > 0 && !suppress))
        return fail(AESIR_ERR_INVALID, "sample_token: bad token list");
    const int64_t n_lists = n_context + n_suppress;
    AESIR_TRY(ensure_work(ctx, vocab, n_lists));
    SamplerWork *w = ctx->sampler;
    hipStream_t s = ctx->stream;
    const bool greedy = cfg->temperature <= 0.0f || cfg->top_k == 1;  // sampler.mojo:235
    if (greedy && n_suppress == 0) {  // the greedy branch reads no penalty state: argmax of the logits
        hipLaunchKernelGGL(sampler_greedy_kernel, dim3(1), dim3(1024), 0, s, (const h16 *)logits, vocab,
                           (const uint8_t *)nullptr, w->result);
        AESIR_LAUNCH_CHECK("sampler_greedy_kernel");
        AESIR_HIP_TRY(hipMemcpyAsync(ctx->pinned_i64, w->result, 16, hipMemcpyDeviceToHost, s));
        AESIR_HIP_TRY(hipStreamSynchronize(s));
        *token = ctx->pinned_i64[0];
        return AESIR_OK;
    }
    if (n_context > 0)
        AESIR_HIP_TRY(hipMemcpyAsync(w->lists, context, (size_t)n_context * 8, hipMemcpyHostToDevice, s));
    if (n_suppress > 0)
        AESIR_HIP_TRY(hipMemcpyAsync(w->lists + n_context, suppress, (size_t)n_suppress * 8, hipMemcpyHostToDevice, s));
    const unsigned g = (unsigned)((vocab + kSThreads - 1) / kSThreads < 4096 ? (vocab + kSThreads - 1) / kSThreads : 4096);
    hipLaunchKernelGGL(sampler_clear_kernel, dim3(g), dim3(kSThreads), 0, s, w->counts, w->mask, vocab);
    AESIR_LAUNCH_CHECK("sampler_clear_kernel");
    if (n_lists > 0) {
        const unsigned gl = (unsigned)((n_lists + kSThreads - 1) / kSThreads < 4096 ? (n_lists + kSThreads - 1) / kSThreads : 4096);
        hipLaunchKernelGGL(sampler_mark_kernel, dim3(gl), dim3(kSThreads), 0, s, w->lists, n_context,
                           w->lists + n_context, n_suppress, w->counts, w->mask, vocab);
        AESIR_LAUNCH_CHECK("sampler_mark_kernel");
    }
    uint64_t st = *rng_state;
    if (greedy) {
        hipLaunchKernelGGL(sampler_greedy_kernel, dim3(1), dim3(1024), 0, s, (const h16 *)logits, vocab, w->mask,
                           w->result);
        AESIR_LAUNCH_CHECK("sampler_greedy_kernel");
    } else {
        SampleParams p{};
        p.repetition_penalty = cfg->repetition_penalty;
        p.frequency_penalty = cfg->frequency_penalty;
        p.presence_penalty = cfg->presence_penalty;
        p.apply_rep = cfg->repetition_penalty != 1.0f && n_context > 0;
        p.apply_freq = !(cfg->frequency_penalty == 0.0f && cfg->presence_penalty == 0.0f) && n_context > 0;
        p.apply_temp = cfg->temperature > 0.0f && cfg->temperature != 1.0f;
        p.inv_temp = 1.0f / cfg->temperature;
        p.top_k = cfg->top_k;
        p.top_p = cfg->top_p;
        p.min_p = cfg->min_p;
        const bool k_on = cfg->top_k > 0 && cfg->top_k < vocab;
        const bool p_on = cfg->top_p < 1.0f && vocab > 1;
        const bool m_on = cfg->min_p > 0.0f && cfg->min_p < 1.0f && vocab > 1;
        p.sort = k_on || p_on || m_on;
        uint64_t peek = st;
        p.u = (float)(rune_next(&peek) & 0xFFFFFFULL) / 16777216.0f;
        hipLaunchKernelGGL(sampler_prepare_kernel, dim3(g), dim3(kSThreads), 0, s, (const h16 *)logits, vocab,
                           w->counts, w->mask, p, w->vals, w->keys, w->idx);
        AESIR_LAUNCH_CHECK("sampler_prepare_kernel");
        if (p.sort) {
            size_t bytes = w->sort_tmp_bytes;
            AESIR_HIP_TRY(rocprim::radix_sort_pairs(w->sort_tmp, bytes, w->keys, w->keys_out, w->idx, w->idx_out,
                                                    (unsigned)vocab, 0, 32, s));
        }
        hipLaunchKernelGGL(sampler_tail_kernel, dim3(1), dim3(kTailThreads), 0, s, w->vals,
                           p.sort ? (const int32_t *)w->idx_out : nullptr, vocab, p, w->marks, w->result);
        AESIR_LAUNCH_CHECK("sampler_tail_kernel");
        st = peek;
    }
    int64_t res[2];
    AESIR_HIP_TRY(hipMemcpyAsync(ctx->pinned_i64, w->result, 16, hipMemcpyDeviceToHost, s));
    AESIR_HIP_TRY(hipStreamSynchronize(s));
    std::memcpy(res, ctx->pinned_i64, 16);
    *token = res[0];
    if (res[1]) *rng_state = st;  // the draw consumed RuneRNG.next_float32
    return AESIR_OK;
}

}  // extern "C"
