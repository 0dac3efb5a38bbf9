// The full sampler stack on the device: sample_token_from_logits (core/sampler.mojo:217-305).
//
//   prepare   one thread per vocabulary entry: sanitize_logit (:9-14), the suppress mask (:197-211),
//             the repetition and frequency / presence penalties (:54-76, :143-163) from a context
//             histogram built with integer atomics (order-independent, so deterministic), and the
//             temperature scale (:79-88); f32 arithmetic in the reference's order
//   sort      when top-k, top-p or min-p truncates: one stable LSD radix sort (rocPRIM) of
//             (descending logit key, index). Equal logits (-0 == +0) keep index order, which is the
//             order the reference's stable insertion sort (:92-104) produces; every later stage of
//             the stack sees an already sorted prefix, so one sort serves all of them. With
//             top_k <= 4096 only that prefix is found: a radix select of the k-th key, an
//             index-order compaction and a sort of the k selected pairs (same order, no full sort)
//   tail      top_k <= 4096: one workgroup makes the truncations and the draw, the running sums
//             of apply_top_p, apply_min_p and the draw in one lane in candidate order (f32
//             addition is not associative; the sums must follow the reference's order to choose
//             the same cut and token), the next LDS tile of exps computed by the other waves
//   chunked   longer candidate lists: each running sum (top-p's sum and cut, min-p's sum, the
//             final draw's sum and walk) is a terms pass and a records pass over the whole device
//             and one wave that reproduces the sequential f32 sum bit for bit, with one integer
//             add per chunk where no rounding depends on the order; the candidate count stays on
//             the device between the stages
//   greedy    temperature <= 0 or top_k == 1: the first maximum of the sanitized, masked logits
//             (per-workgroup maxima over strided ranges, then one workgroup)
//
// The random number comes from RuneRNG on the host (one draw per sampled token, consumed only
// when the reference consumes it: a final sum that is not <= 0, NaN included). exp is evaluated as the correctly
// rounded f32 value (f64 exp rounded once) so that the CPU oracle computes the same bits.
#include <cstring>
#include <rocprim/device/device_radix_sort.hpp>

#include "common.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aesir {

constexpr int kSThreads = 256;
constexpr int kTailThreads = 256;
constexpr int kSeqTile = 4096;  // terms per LDS tile of the tail (two tiles); its candidate limit

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

// Clears the context histogram and suppress flags, and the top-k selection's key histograms.
__global__ void sampler_clear_kernel(int32_t *__restrict__ counts, uint8_t *__restrict__ mask, int64_t V,
                                     uint32_t *__restrict__ hist, int nhist) {
    const int64_t t0 = (int64_t)blockIdx.x * kSThreads + threadIdx.x, step = (int64_t)gridDim.x * kSThreads;
    for (int64_t i = t0; i < V; i += step) {
        counts[i] = 0;
        mask[i] = 0;
    }
    for (int64_t i = t0; i < nhist; i += step) hist[i] = 0;
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

// ------------------------------------------------------------------ top-k selection
//
// With top_k <= kSeqTile only the first top_k candidates of the stable descending sort are ever
// read, so instead of sorting the vocabulary the stages find them exactly:
//   1. the k-th smallest radix key T (ascending key order is the sort's order) by a radix select,
//      three histogram passes over the key's digits (bits 21-31, 10-20, 0-9); pass p counts the
//      keys that match the digits already fixed, each workgroup deriving those digits from the
//      earlier passes' histograms (a scan of 2048 bins per pass)
//   2. per workgroup, the counts of keys below T and equal to T; then the compaction, in index
//      order: every key below T, and the lowest-index keys equal to T that complete top_k (the
//      stable sort keeps equal keys in index order)
//   3. one workgroup sorts the top_k (key, index) pairs as 64-bit values in LDS (bitonic); the
//      pairs are distinct, so any correct sort gives the stable sort's order
constexpr int kSelBins = 2048;
constexpr int kSelPer = 4;                              // keys per thread of the selection passes
constexpr int kSelBlock = kSThreads * kSelPer;          // keys per workgroup
constexpr int kSelShift[3] = {21, 10, 0};
constexpr uint32_t kSelMask[3] = {0x7FFu, 0x7FFu, 0x3FFu};

struct SelState {
    uint32_t prefix;  // digits fixed so far
    uint32_t rank;    // 1-based rank of the wanted key among the keys matching prefix
    uint32_t lt;      // keys below every key matching prefix
};

// The digits fixed by passes 0 .. np-1, from their histograms (the whole workgroup takes part).
__device__ SelState sel_state(const uint32_t *__restrict__ hist, int np, uint32_t k, uint32_t *sh) {
    SelState st{0u, k, 0u};
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int per = kSelBins / kSThreads;  // 8 bins per thread
    for (int q = 0; q < np; q++) {
        const uint32_t *h = hist + q * kSelBins;
        uint32_t v[per], sum = 0;
#pragma unroll
        for (int j = 0; j < per; j++) {
            v[j] = h[tid * per + j];
            sum += v[j];
        }
        // exclusive prefix of the thread sums over the workgroup
        uint32_t incl = sum;
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t t = __shfl_up(incl, o);
            if (lane >= o) incl += t;
        }
        if (lane == 63) sh[wave] = incl;
        __syncthreads();
        uint32_t base = 0;
        for (int w = 0; w < wave; w++) base += sh[w];
        uint32_t c = base + incl - sum;  // keys in bins before this thread's
        if (c < st.rank && st.rank <= c + sum) {
            uint32_t d = 0;
#pragma unroll
            for (int j = 0; j < per; j++) {
                if (c + v[j] >= st.rank) {
                    d = (uint32_t)(tid * per + j);
                    break;
                }
                c += v[j];
            }
            sh[4] = d;
            sh[5] = c;
        }
        __syncthreads();
        const uint32_t d = sh[4], before = sh[5];
        st.lt += before;
        st.rank -= before;
        st.prefix |= d << kSelShift[q];
        __syncthreads();
    }
    return st;
}

__device__ __forceinline__ bool sel_match(uint32_t key, const SelState &st, int np) {
    return np == 0 || (key >> kSelShift[np - 1]) == (st.prefix >> kSelShift[np - 1]);
}

template <int NP>
__global__ __launch_bounds__(kSThreads) void sampler_select_hist_kernel(const uint32_t *__restrict__ keys, int64_t V,
                                                                        uint32_t *__restrict__ hist, uint32_t k) {
    __shared__ uint32_t lh[kSelBins];
    __shared__ uint32_t sh[8];
    const int tid = threadIdx.x;
    for (int b = tid; b < kSelBins; b += kSThreads) lh[b] = 0;
    const SelState st = sel_state(hist, NP, k, sh);
    __syncthreads();  // lh is clear (sel_state synchronizes only when NP > 0)
    const int64_t base = (int64_t)blockIdx.x * kSelBlock;
#pragma unroll
    for (int j = 0; j < kSelPer; j++) {
        const int64_t i = base + j * kSThreads + tid;
        if (i < V) {
            const uint32_t key = keys[i];
            if (sel_match(key, st, NP)) atomicAdd(&lh[(key >> kSelShift[NP]) & kSelMask[NP]], 1u);
        }
    }
    __syncthreads();
    uint32_t *gh = hist + NP * kSelBins;
    for (int b = tid; b < kSelBins; b += kSThreads)
        if (lh[b]) atomicAdd(&gh[b], lh[b]);
}

// Per workgroup of kSelBlock keys: how many are below T and how many equal it.
__global__ __launch_bounds__(kSThreads) void sampler_select_count_kernel(const uint32_t *__restrict__ keys, int64_t V,
                                                                         const uint32_t *__restrict__ hist, uint32_t k,
                                                                         uint32_t *__restrict__ cnt) {
    __shared__ uint32_t sh[8];
    __shared__ uint32_t red[2][kSThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const SelState st = sel_state(hist, 3, k, sh);
    const uint32_t T = st.prefix;
    const int64_t base = (int64_t)blockIdx.x * kSelBlock;
    uint32_t lt = 0, eq = 0;
#pragma unroll
    for (int j = 0; j < kSelPer; j++) {
        const int64_t i = base + j * kSThreads + tid;
        if (i < V) {
            const uint32_t key = keys[i];
            lt += key < T;
            eq += key == T;
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        lt += __shfl_xor(lt, o);
        eq += __shfl_xor(eq, o);
    }
    if (lane == 0) {
        red[0][wave] = lt;
        red[1][wave] = eq;
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t a = 0, b = 0;
        for (int w = 0; w < kSThreads / 64; w++) {
            a += red[0][w];
            b += red[1][w];
        }
        cnt[2 * blockIdx.x] = a;
        cnt[2 * blockIdx.x + 1] = b;
    }
}

// The compaction: key-below-T entries at their index-order rank among them, the first
// `rank` equal-key entries (in index order) after them; 64-bit (key, index) values.
__global__ __launch_bounds__(kSThreads) void sampler_select_compact_kernel(const uint32_t *__restrict__ keys, int64_t V,
                                                                           const uint32_t *__restrict__ hist, uint32_t k,
                                                                           const uint32_t *__restrict__ cnt,
                                                                           uint64_t *__restrict__ cand) {
    __shared__ uint32_t sh[8];
    __shared__ uint32_t wl[kSThreads / 64], we[kSThreads / 64];
    __shared__ uint32_t pre_s[2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const SelState st = sel_state(hist, 3, k, sh);
    const uint32_t T = st.prefix, need = st.rank, total_lt = st.lt;
    // keys below T and equal to T in the workgroups before this one
    {
        uint32_t a = 0, b = 0;
        for (int w = tid; w < (int)blockIdx.x; w += kSThreads) {
            a += cnt[2 * w];
            b += cnt[2 * w + 1];
        }
        for (int o = 32; o > 0; o >>= 1) {
            a += __shfl_xor(a, o);
            b += __shfl_xor(b, o);
        }
        if (lane == 0) {
            wl[wave] = a;
            we[wave] = b;
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t x = 0, y = 0;
            for (int w = 0; w < kSThreads / 64; w++) {
                x += wl[w];
                y += we[w];
            }
            pre_s[0] = x;
            pre_s[1] = y;
        }
        __syncthreads();
    }
    uint32_t run_lt = pre_s[0], run_eq = pre_s[1];
    const int64_t base = (int64_t)blockIdx.x * kSelBlock;
    for (int j = 0; j < kSelPer; j++) {  // index order: pass j covers keys base + j * 256 + [0, 256)
        const int64_t i = base + j * kSThreads + tid;
        const uint32_t key = i < V ? keys[i] : 0xFFFFFFFFu;
        const bool is_lt = i < V && key < T, is_eq = i < V && key == T;
        const uint64_t bl = __ballot(is_lt), be = __ballot(is_eq);
        const uint32_t rl = (uint32_t)__popcll(bl & ((1ull << lane) - 1ull));
        const uint32_t re = (uint32_t)__popcll(be & ((1ull << lane) - 1ull));
        __syncthreads();  // wl / we of the previous pass have been read
        if (lane == 0) {
            wl[wave] = (uint32_t)__popcll(bl);
            we[wave] = (uint32_t)__popcll(be);
        }
        __syncthreads();
        uint32_t ol = run_lt, oe = run_eq;
        for (int w = 0; w < wave; w++) {
            ol += wl[w];
            oe += we[w];
        }
        // the slots stay below k by construction (total_lt + need = k); the bounds are checked anyway
        if (is_lt && ol + rl < k) cand[ol + rl] = ((uint64_t)key << 32) | (uint64_t)i;
        if (is_eq && oe + re < need && total_lt + oe + re < k)
            cand[total_lt + oe + re] = ((uint64_t)key << 32) | (uint64_t)i;
        for (int w = 0; w < kSThreads / 64; w++) {
            run_lt += wl[w];
            run_eq += we[w];
        }
    }
}

// Sorts the k <= kSeqTile selected (key, index) values (bitonic, in LDS) and writes the indices.
constexpr int kSelSortThreads = 1024;
__global__ __launch_bounds__(kSelSortThreads) void sampler_select_sort_kernel(const uint64_t *__restrict__ cand,
                                                                              int k, int32_t *__restrict__ order) {
    __shared__ uint64_t v[kSeqTile];
    int m = 1;
    while (m < k) m <<= 1;
    for (int i = threadIdx.x; i < m; i += kSelSortThreads) v[i] = i < k ? cand[i] : ~0ull;
    __syncthreads();
    for (int size = 2; size <= m; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < m; i += kSelSortThreads) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool up = (i & size) == 0;
                    const uint64_t a = v[i], b = v[j];
                    if ((a > b) == up) {
                        v[i] = b;
                        v[j] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    for (int i = threadIdx.x; i < k; i += kSelSortThreads) order[i] = (int32_t)(v[i] & 0xFFFFFFFFull);
}

// Greedy branch (:241-261): best = 0, max = value of index 0, strict '>' ascending; values are
// sanitized and suppressed ones are -1e9. Equivalent to the lowest index of the maximum, which two
// launches find: kGreedyParts workgroups take strided ranges of the logits (each thread sees its
// indices in increasing order, so strict '>' keeps its first maximum) and reduce them to one
// (value, index) pair each, the larger value winning and equal values going to the lower index;
// one workgroup then reduces the pairs the same way.
constexpr int kGreedyParts = 128;
constexpr int kGreedyThreads = 256;

__device__ __forceinline__ void greedy_pick(float &bv, int64_t &bi, float v, int64_t i) {
    if (i >= 0 && (bi < 0 || v > bv || (v == bv && i < bi))) {
        bv = v;
        bi = i;
    }
}

__device__ __forceinline__ void greedy_block_reduce(float &bv, int64_t &bi, float *sv, int64_t *si) {
    for (int o = 32; o > 0; o >>= 1) {
        const float v = __shfl_xor(bv, o);
        const int64_t i = __shfl_xor(bi, o);
        greedy_pick(bv, bi, v, i);
    }
    const int w = threadIdx.x / 64;
    if ((threadIdx.x & 63) == 0) {
        sv[w] = bv;
        si[w] = bi;
    }
    __syncthreads();
    bv = sv[0];
    bi = si[0];
    for (int k = 1; k < kGreedyThreads / 64; k++) greedy_pick(bv, bi, sv[k], si[k]);
}

__global__ __launch_bounds__(kGreedyThreads) void sampler_greedy_part_kernel(const h16 *__restrict__ logits, int64_t V,
                                                                             const uint8_t *__restrict__ mask,
                                                                             float *__restrict__ pv,
                                                                             int64_t *__restrict__ pi) {
    __shared__ float sv[kGreedyThreads / 64];
    __shared__ int64_t si[kGreedyThreads / 64];
    float bv = -INFINITY;
    int64_t bi = -1;
    for (int64_t i = (int64_t)blockIdx.x * kGreedyThreads + threadIdx.x; i < V;
         i += (int64_t)gridDim.x * kGreedyThreads) {
        float v = sanitize_logit((float)logits[i]);
        if (mask && mask[i]) v = -1e9f;
        if (bi < 0 || v > bv) {
            bv = v;
            bi = i;
        }
    }
    greedy_block_reduce(bv, bi, sv, si);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

__global__ __launch_bounds__(kGreedyThreads) void sampler_greedy_finish_kernel(const float *__restrict__ pv,
                                                                               const int64_t *__restrict__ pi,
                                                                               int nparts, int64_t *out) {
    __shared__ float sv[kGreedyThreads / 64];
    __shared__ int64_t si[kGreedyThreads / 64];
    float bv = -INFINITY;
    int64_t bi = -1;
    for (int k = threadIdx.x; k < nparts; k += kGreedyThreads) greedy_pick(bv, bi, pv[k], pi[k]);
    greedy_block_reduce(bv, bi, sv, si);
    if (threadIdx.x == 0) {
        out[0] = bi < 0 ? 0 : bi;
        out[1] = 0;  // no random number consumed
    }
}

// Truncations and the draw over at most kSeqTile candidates (top_k <= kSeqTile), in one
// workgroup: value i is vals[order ? order[i] : i]. The running f32 sums of apply_top_p and
// apply_min_p are evaluated in candidate order by lane 0 of wave 0 (f32 addition is not
// associative, so the order fixes the cut). The terms come from two LDS tiles: while lane 0 adds
// one tile, waves 1-3 compute the next tile's terms into the other. Longer candidate lists take
// the chunked stages below.
constexpr int kSeqBlock = 32;   // terms per block of lane 0's adds

// Lane 0's adds over one tile, acc += buf[e] for e in [0, cnt), 32 terms per block with the next
// block's LDS reads in flight. kHit: stops at the first e with target <= acc (returned in hit,
// -1 when none); a block is added first and re-added term by term only when the target falls
// inside it (terms are >= 0, so acc never decreases).
template <bool kHit>
__device__ __forceinline__ float chain_tile(const float *buf, int cnt, float acc, float target, int &hit) {
    const int nb = cnt / kSeqBlock;
    f32x4 ra[8], rb[8];
    auto load = [&](f32x4(&r)[8], int b) {
#pragma unroll
        for (int q = 0; q < 8; q++) r[q] = *reinterpret_cast<const f32x4 *>(&buf[kSeqBlock * b + 4 * q]);
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
                        hit = kSeqBlock * b + 4 * q + u;
                        acc = c;
                        return true;
                    }
                }
        }
        acc = a;
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
    for (int e = kSeqBlock * nb; e < cnt; e++) {  // the short last block of the last tile
        acc += buf[e];
        if (kHit && target <= acc) {
            hit = e;
            return acc;
        }
    }
    return acc;
}

// acc_i = acc_{i-1} + term(i) in f32 over i in [0, m), m >= 1, in index order. Returns the first
// i with target <= acc_i (m when none) under kHit, else m; the running sum where the chain
// stopped goes to total (every thread). Enter and leave with the workgroup converged;
// tile0/tile1 and n_sh/f_sh are free on entry.
template <bool kHit, class Term>
__device__ __forceinline__ int64_t ordered_chain(float *tile0, float *tile1, int64_t m, Term term, float target,
                                                 float &total, int64_t *n_sh, float *f_sh) {
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
                acc = chain_tile<kHit>(cur, tile_cnt(k), acc, target, he);
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

// Device-side state of the chunked stages: the candidate count as the truncations leave it, the
// count of chunks a records pass lists as likely slow, the last sum pass's total and min-p's first
// failing index.
struct DrawHdr {
    int64_t n;
    uint32_t n_slow;
    float sum;
    int64_t kept;
};

__global__ __launch_bounds__(kTailThreads) void sampler_tail_kernel(const float *__restrict__ vals,
                                                                    const int32_t *__restrict__ order, int64_t V,
                                                                    SampleParams p, int64_t *out) {
    __shared__ __align__(16) float tile[2][kSeqTile];
    __shared__ float red[kTailThreads];
    __shared__ int64_t n_sh[2];
    __shared__ float f_sh;
    const int tid = threadIdx.x;
    auto val = [&](int64_t i) -> float { return vals[order ? order[i] : i]; };
    int64_t n = V;
    if (p.top_k > 0 && p.top_k < n) n = p.top_k;  // apply_top_k (:107-116)

    if (p.top_p < 1.0f && n > 1) {  // apply_top_p (:119-147): exps relative to the first (largest) logit
        const float mx = val(0);
        float sum, stop;
        ordered_chain<false>(tile[0], tile[1], n, [&](int64_t i) { return exp_f32(val(i) - mx); }, 0.0f, sum, n_sh,
                             &f_sh);
        const int64_t cut = ordered_chain<true>(
            tile[0], tile[1], n,
            [&](int64_t i) {
                const float e = exp_f32(val(i) - mx);
                return sum > 0.0f ? e / sum : e;
            },
            p.top_p, stop, n_sh, &f_sh);
        n = cut < n ? cut + 1 : n;
    }
    if (p.min_p > 0.0f && p.min_p < 1.0f && n > 1) {  // apply_min_p (:166-194)
        const float mx = val(0);
        float sum;
        ordered_chain<false>(tile[0], tile[1], n, [&](int64_t i) { return exp_f32(val(i) - mx); }, 0.0f, sum, n_sh,
                             &f_sh);
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
    // At most kSeqTile candidates: the final draw (:284-305) here, its exps in one LDS tile and
    // both running sums (sum_e, then the inverse-CDF walk) in lane 0 in candidate order.
    float mx = -INFINITY;
    for (int64_t i = tid; i < n; i += kTailThreads) mx = fmaxf(mx, val(i));
    red[tid] = mx;
    __syncthreads();
    for (int st = kTailThreads / 2; st > 0; st >>= 1) {
        if (tid < st) red[tid] = fmaxf(red[tid], red[tid + st]);
        __syncthreads();
    }
    mx = red[0];
    for (int e = tid; e < (int)n; e += kTailThreads) tile[0][e] = exp_f32(val(e) - mx);
    __syncthreads();
    if (tid == 0) {
        int he;
        const float sum_e = chain_tile<false>(tile[0], (int)n, 0.0f, 0.0f, he);
        if (sum_e <= 0.0f) {  // a NaN sum goes on to the walk, as in the reference
            out[0] = order ? order[0] : 0;
            out[1] = 0;
        } else {
            const float r = p.u * sum_e;
            chain_tile<true>(tile[0], (int)n, 0.0f, r, he);
            const int64_t pick = he >= 0 ? he : n - 1;
            out[0] = order ? order[pick] : pick;
            out[1] = 1;
        }
    }
}

// ------------------------------------------------------------------ the final draw (:284-305)
//
// max over the candidates, e_i = exp(x_i - max), sum_e = the f32 running sum of the e_i in
// candidate order, r = u * sum_e, and the first i whose running sum reaches r.
//
// The running sum acc_i = fl(acc_{i-1} + e_i) is evaluated exactly without one add per term. While
// acc stays in one binade [2^E, 2^(E+1)) its bit pattern counts ulps u = 2^(E-23), and for a term
// e >= 0, fl(acc + e) = acc + RN(e / u) ulps, unless e / u lies exactly halfway between two
// integers (the parity of acc then decides) or the result leaves the binade. So for a block of
// terms and a binade E, K_E = sum RN(e / u) is the exact advance of acc's bit pattern whenever acc
// enters the block in binade E, no term of the block is a halfway case for E and mantissa(acc) +
// K_E < 2^23, i.e. whenever acc's bits lie in [E's first pattern, E's last pattern - K_E]. These
// increments are computed for every block in parallel for the two binades that an f64 estimate of
// the running sum puts the chunk in (E_a and E_a + 1); one wave then walks the chunks in order,
// advancing acc by one range test and one integer add per chunk where the conditions hold, else
// per 32-term block, else by re-adding the block's terms one by one. Every value it produces is
// the sequential sum's value at that index, bit for bit. The running sum at the start of every
// batch of kBatch chunks is recorded; the draw's walk (the same terms in the same order, so the
// same running sums) finds its batch from these in parallel, steps through at most kBatch chunks
// of it the same way, and re-adds one chunk term by term.
constexpr int kDrawThreads = 256;
constexpr int kDrawChunk = 256;                      // terms per chunk (one workgroup of the parallel kernels)
constexpr int kDrawSub = 32;                         // terms per block inside a chunk
constexpr int kDrawSubs = kDrawChunk / kDrawSub;     // 8
constexpr int kHeadWords = 8;                        // per chunk: lo, span, K for E_a and E_a + 1; E_a; flags
constexpr int kBlockWords = 6;                       // per block: lo, span, K for E_a and E_a + 1
constexpr int kSubWords = kBlockWords * kDrawSubs;   // per chunk: its blocks' ranges (48 words)
constexpr int kBatch = 64 / kHeadWords;              // chunk headers per vector load of the walk (8)
constexpr int kRoundBatches = 64;                    // header batches staged in LDS per round of the walk
constexpr int kStage = 32;                           // likely-slow chunks staged in LDS for the walk (<= 64)
constexpr int kNoBinade = -1000;                     // E_a of a chunk without an estimate
constexpr uint32_t kUlpCap = 1u << 24;               // saturated increment (fails every mantissa check)
constexpr uint32_t kLikelySlow = 1u << 16;           // header flag: the chunk may need its blocks
constexpr int kSlowListMax = 4096;                   // likely-slow chunk ids the records kernel lists
static_assert(kDrawThreads == kDrawChunk, "one thread per term of a chunk");
static_assert(kDrawSubs <= 8, "block flags take 8 bits per binade");

__device__ __forceinline__ float block_max_f32(float v, float *sh) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int w = threadIdx.x / 64;
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    v = sh[0];
    for (int k = 1; k < kDrawThreads / 64; k++) v = fmaxf(v, sh[k]);
    __syncthreads();
    return v;
}

__device__ __forceinline__ double block_sum_f64(double v, double *sh) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x / 64;
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    v = sh[0];
    for (int k = 1; k < kDrawThreads / 64; k++) v += sh[k];
    __syncthreads();
    return v;
}

// Per-chunk maxima of the candidates (fmaxf: a NaN candidate is skipped here, and it makes sum_e
// NaN whatever the maximum, as it does in the reference).
__global__ __launch_bounds__(kDrawThreads) void sampler_chunk_max_kernel(const float *__restrict__ vals,
                                                                         const int32_t *__restrict__ order,
                                                                         const DrawHdr *__restrict__ hdr,
                                                                         float *__restrict__ cmax) {
    __shared__ float sh[kDrawThreads / 64];
    const int64_t n = hdr->n;
    const int64_t base = (int64_t)blockIdx.x * kDrawChunk;
    if (base >= n) return;
    const int64_t i = base + threadIdx.x;
    float v = -INFINITY;
    if (i < n) v = vals[order ? order[i] : i];
    v = block_max_f32(v, sh);
    if (threadIdx.x == 0) cmax[blockIdx.x] = v;
}

// The terms of one chunk of a running sum, and the chunk's f64 sum (an estimate for the binades):
//   kTermsDraw   e_i = exp(x_i - max), max over the chunk maxima (the final draw, :284-293)
//   kTermsExp    e_i = exp(x_i - x_0), x_0 the first (largest) candidate (apply_top_p :128-134,
//                apply_min_p :175-181)
//   kTermsProb   p_i = e_i / sum (e_i when sum <= 0), sum the previous pass's total (:136-138)
// The truncation modes do nothing for one candidate or fewer (the reference returns early). Block
// 0 also clears the likely-slow count for the records pass that follows.
enum { kTermsDraw, kTermsExp, kTermsProb };
template <int MODE>
__global__ __launch_bounds__(kDrawThreads) void sampler_terms_kernel(const float *__restrict__ vals,
                                                                     const int32_t *__restrict__ order,
                                                                     DrawHdr *__restrict__ hdr,
                                                                     const float *__restrict__ cmax,
                                                                     float *__restrict__ terms,
                                                                     double *__restrict__ csum) {
    __shared__ float shf[kDrawThreads / 64];
    __shared__ double shd[kDrawThreads / 64];
    const int64_t n = hdr->n;
    const int64_t base = (int64_t)blockIdx.x * kDrawChunk;
    if (MODE != kTermsDraw && n <= 1) return;
    if (base >= n) return;
    if (blockIdx.x == 0 && threadIdx.x == 0) hdr->n_slow = 0;
    auto val = [&](int64_t i) -> float { return vals[order ? order[i] : i]; };
    float mx;
    if constexpr (MODE == kTermsDraw) {
        const int64_t nch = (n + kDrawChunk - 1) / kDrawChunk;
        mx = -INFINITY;
        for (int64_t c = threadIdx.x; c < nch; c += kDrawThreads) mx = fmaxf(mx, cmax[c]);
        mx = block_max_f32(mx, shf);
    } else {
        mx = val(0);
    }
    const int64_t i = base + threadIdx.x;
    float t = 0.0f;
    if (i < n) {
        t = exp_f32(val(i) - mx);
        if constexpr (MODE == kTermsProb) {
            const float sum = hdr->sum;
            t = sum > 0.0f ? t / sum : t;
        }
        terms[i] = t;
    }
    const double s = block_sum_f64((double)t, shd);
    if (threadIdx.x == 0) csum[blockIdx.x] = s;
}

// The first candidate count of the chunked stages: top_k's cut (:107-116) or the vocabulary.
__global__ void sampler_set_n_kernel(DrawHdr *hdr, int64_t n) {
    hdr->n = n;
    hdr->n_slow = 0;
}

// apply_min_p's cut (:183-194) after its sum pass: p_i = e_i / sum (e_i when sum <= 0) against
// min_p * p_0. The probabilities never increase along the sorted candidates, so the kept ones are
// the prefix before the first failing index, which the workgroups find with an atomic minimum.
__global__ __launch_bounds__(kDrawThreads) void sampler_minp_cut_kernel(const float *__restrict__ vals,
                                                                        const int32_t *__restrict__ order,
                                                                        DrawHdr *__restrict__ hdr, float min_p) {
    __shared__ int64_t first_s;
    const int64_t n = hdr->n;
    const int64_t base = (int64_t)blockIdx.x * kDrawChunk;
    if (n <= 1 || base >= n) return;
    if (threadIdx.x == 0) first_s = n;
    __syncthreads();
    const float sum = hdr->sum;
    const float mx = vals[order[0]];
    const float e0 = exp_f32(0.0f);  // the first candidate's exp (x_0 - x_0 = 0)
    const float p0 = sum > 0.0f ? e0 / sum : e0;
    const float threshold = min_p * p0;
    const int64_t i = base + threadIdx.x;
    if (i < n) {
        const float e = exp_f32(vals[order[i]] - mx);
        const float pr = sum > 0.0f ? e / sum : e;
        if (!(pr >= threshold)) atomicMin(reinterpret_cast<unsigned long long *>(&first_s), (unsigned long long)i);
    }
    __syncthreads();
    if (threadIdx.x == 0 && first_s < n)
        atomicMin(reinterpret_cast<unsigned long long *>(&hdr->kept), (unsigned long long)first_s);
}

// n = the kept prefix when it is not empty (:196-197).
__global__ void sampler_minp_finish_kernel(DrawHdr *hdr) {
    const int64_t n = hdr->n, kept = hdr->kept;
    if (n > 1 && kept > 0 && kept < n) hdr->n = kept;
}

// RN(t / 2^(E-23)) for E in [-100, 101], with the halfway flag. NaN, infinite or negative terms
// are flagged so that their block is re-added; increments of 2^24 or more saturate.
__device__ __forceinline__ uint32_t ulps_of(float t, int E, bool &half) {
    if (!(t >= 0.0f) || isinf(t)) {
        half = true;
        return kUlpCap;
    }
    const double x = ldexp((double)t, 23 - E);
    half = false;
    if (x >= 16777216.0) return kUlpCap;
    const double f = floor(x);
    const double r = x - f;  // exact: x carries at most 24 significant bits
    half = r == 0.5;
    return (uint32_t)f + (r > 0.5 ? 1u : 0u);
}

// One chunk's header and its blocks' ranges. E_a comes from the f64 running-sum estimate at
// the chunk's start, shifted down by 1/64 so that E_a or E_a + 1 holds the true sum (the
// sequential f32 sum of k terms is within k * 2^-24 of the exact one). Header: for E_a and
// E_a + 1, the first bit pattern lo, the span of patterns from which the chunk-wide increment K
// applies, and K (an empty range, lo = 0xFFFFFFFF with span 0 and K 0, when a halfway term or the
// missing estimate rules the binade out); then E_a; then the blocks' halfway flags (bits 0-7 for
// E_a, 8-15 for E_a + 1) and kLikelySlow when the estimate over the chunk, widened by its typical
// error (2^-12), straddles a binade boundary (or there is no estimate, or a halfway term); such a
// chunk is also appended to slow_list (any order), which only decides what the walk stages in
// LDS. Each 32-term block gets the same six words for its own increments.
__global__ __launch_bounds__(kDrawThreads) void sampler_records_kernel(const float *__restrict__ terms,
                                                                       const double *__restrict__ csum,
                                                                       DrawHdr *__restrict__ hdr_rw,
                                                                       uint32_t *__restrict__ heads,
                                                                       uint32_t *__restrict__ subk,
                                                                       uint32_t *__restrict__ slow_list) {
    __shared__ double shd[kDrawThreads / 64];
    __shared__ uint32_t ka_s[kDrawSubs], kb_s[kDrawSubs], half_s[kDrawSubs];
    const int64_t n = hdr_rw->n;
    const int64_t base = (int64_t)blockIdx.x * kDrawChunk;
    if (base >= n) return;
    const int tid = threadIdx.x;
    double s = 0.0;
    for (int64_t c = tid; c < (int64_t)blockIdx.x; c += kDrawThreads) s += csum[c];
    s = block_sum_f64(s, shd);
    const double s_end = s + csum[blockIdx.x];
    int Ea = kNoBinade;
    bool straddle = true;
    if (s > 0.0 && s < 1e30) {
        const int e = ilogb(s * (1.0 - 1.0 / 64));
        if (e >= -100 && e <= 100) {
            Ea = e;
            straddle = !(s_end < 1e30) || ilogb(s * (1.0 - 1.0 / 4096)) != ilogb(s_end * (1.0 + 1.0 / 4096));
        }
    }
    uint32_t qa = 0, qb = 0;
    bool ha = false, hb = false;
    const int64_t i = base + tid;
    if (i < n && Ea != kNoBinade) {
        const float t = terms[i];
        qa = ulps_of(t, Ea, ha);
        qb = ulps_of(t, Ea + 1, hb);
    }
    // 32-term blocks are half waves: sums (each term <= 2^24, so a block < 2^29) and flags
    for (int o = 16; o > 0; o >>= 1) {
        qa += __shfl_xor(qa, o);
        qb += __shfl_xor(qb, o);
    }
    const uint64_t ba = __ballot(ha), bb = __ballot(hb);
    const int lane = tid & 63;
    if ((lane & 31) == 0) {
        const int sb = tid / kDrawSub;
        const uint32_t ka = qa < kUlpCap ? qa : kUlpCap, kb = qb < kUlpCap ? qb : kUlpCap;
        const bool half_a = (uint32_t)(ba >> lane) != 0u, half_b = (uint32_t)(bb >> lane) != 0u;
        ka_s[sb] = ka;
        kb_s[sb] = kb;
        half_s[sb] = (half_a ? 1u : 0u) | (half_b ? 2u : 0u);
        const bool ok_a = Ea != kNoBinade && !half_a && ka <= 0x7FFFFFu;
        const bool ok_b = Ea != kNoBinade && !half_b && kb <= 0x7FFFFFu;
        uint32_t *r = subk + (int64_t)blockIdx.x * kSubWords + sb * kBlockWords;
        r[0] = ok_a ? (uint32_t)(Ea + 127) << 23 : 0xFFFFFFFFu;
        r[1] = ok_a ? 0x7FFFFFu - ka : 0u;
        r[2] = ok_a ? ka : 0u;
        r[3] = ok_b ? (uint32_t)(Ea + 128) << 23 : 0xFFFFFFFFu;
        r[4] = ok_b ? 0x7FFFFFu - kb : 0u;
        r[5] = ok_b ? kb : 0u;
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t ka = 0, kb = 0, fl = 0;
        for (int k = 0; k < kDrawSubs; k++) {
            ka += ka_s[k];
            kb += kb_s[k];
            fl |= (half_s[k] & 1u) << k;
            fl |= ((half_s[k] >> 1) & 1u) << (8 + k);
        }
        const bool ok_a = Ea != kNoBinade && (fl & 0xFFu) == 0u && ka <= 0x7FFFFFu;
        const bool ok_b = Ea != kNoBinade && (fl & 0xFF00u) == 0u && kb <= 0x7FFFFFu;
        if (straddle || (fl & 0xFFFFu) != 0u) {
            fl |= kLikelySlow;
            const uint32_t k = atomicAdd(&hdr_rw->n_slow, 1u);
            if (k < (uint32_t)kSlowListMax) slow_list[k] = blockIdx.x;
        }
        uint32_t *h = heads + (int64_t)blockIdx.x * kHeadWords;
        h[0] = ok_a ? (uint32_t)(Ea + 127) << 23 : 0xFFFFFFFFu;
        h[1] = ok_a ? 0x7FFFFFu - ka : 0u;
        h[2] = ok_a ? ka : 0u;
        h[3] = ok_b ? (uint32_t)(Ea + 128) << 23 : 0xFFFFFFFFu;
        h[4] = ok_b ? 0x7FFFFFu - kb : 0u;
        h[5] = ok_b ? kb : 0u;
        h[6] = (uint32_t)Ea;
        h[7] = fl;
    }
}

// The walk, then one of: the total (kWalkSum: to hdr->sum, with hdr->kept reset for min-p);
// apply_top_p's cut (kWalkCut: the first i whose running sum of probabilities reaches top_p,
// hdr->n = i + 1, or unchanged when there is none, :140-147); or the final draw (kWalkDraw).
// The walk goes round by round, kRoundBatches batches of kBatch chunks
// at a time. For each round the workgroup stages the chunk headers in LDS, reduces every batch to
// one header of the same form (a range and an increment for each binade, valid when every chunk
// of the batch has one for the first chunk's binade; the chunks' tests then all hold exactly when
// the batch's holds), and stages the block ranges and terms of the round's chunks on the
// likely-slow list.
// Wave 0 then walks the round on scalar registers: a batch header or a chunk's header is read into
// one VGPR, one word per lane, and taken apart with readlane.
enum { kWalkSum, kWalkCut, kWalkDraw };
template <int MODE>
__global__ __launch_bounds__(kDrawThreads) void sampler_draw_kernel(const float *__restrict__ terms,
                                                                    const uint32_t *__restrict__ heads,
                                                                    const uint32_t *__restrict__ subk,
                                                                    const uint32_t *__restrict__ slow_list,
                                                                    DrawHdr *__restrict__ hdr,
                                                                    const int32_t *__restrict__ order,
                                                                    float target_arg, uint32_t *__restrict__ marks,
                                                                    int64_t *__restrict__ out) {
    constexpr int kRoundWords = kRoundBatches * 64;
    __shared__ __align__(16) uint32_t rh[kRoundWords];
    __shared__ uint32_t ragg[kRoundBatches * kHeadWords];
    __shared__ __align__(16) float st_terms[kStage * kDrawChunk];
    __shared__ uint32_t st_subk[kStage * kSubWords];
    __shared__ int st_id[kStage];
    __shared__ __align__(16) float tile[kDrawChunk];
    __shared__ int st_n, wcnt[kDrawThreads / 64];
    __shared__ uint32_t sum_bits, start_bits;
    __shared__ int64_t chunk_s;
    __shared__ int64_t cnt_s[kDrawThreads / 64];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int lane = tid & 63;
    const int64_t n = hdr->n;
    if (MODE != kWalkDraw && n <= 1) return;  // the truncations leave one candidate alone
    const int64_t nch = (n + kDrawChunk - 1) / kDrawChunk;
    const int64_t nbat = (nch + kBatch - 1) / kBatch;  // heads holds nbat whole batches
    const int n_list = (int)(hdr->n_slow < (uint32_t)kSlowListMax ? hdr->n_slow : (uint32_t)kSlowListMax);

    // Stages round b0's headers, batch headers and likely-slow chunks; returns the batch count.
    auto stage_round = [&](int64_t b0) -> int {
        const int nb = (int)(nbat - b0 < kRoundBatches ? nbat - b0 : kRoundBatches);
        const int64_t c_lo = b0 * kBatch, c_hi = (b0 + nb) * kBatch;
        uint32_t first_ids = tid < n_list ? slow_list[tid] : 0xFFFFFFFFu;  // in flight with the headers
        {  // headers: independent 16-byte loads, all in flight together
            const u32x4 *src = reinterpret_cast<const u32x4 *>(heads + b0 * 64);
            u32x4 *dst = reinterpret_cast<u32x4 *>(rh);
            constexpr int kPer = kRoundWords / 4 / kDrawThreads;
            u32x4 v[kPer];
#pragma unroll
            for (int j = 0; j < kPer; j++) {
                const int k = j * kDrawThreads + tid;
                if (k < nb * 16) v[j] = src[k];
            }
#pragma unroll
            for (int j = 0; j < kPer; j++) {
                const int k = j * kDrawThreads + tid;
                if (k < nb * 16) dst[k] = v[j];
            }
        }
        if (tid == 0) st_n = 0;
        __syncthreads();
        // batch headers, one wave per batch; lane = chunk q * kHeadWords + word w
        const int w = lane & (kHeadWords - 1), q = lane / kHeadWords;
        for (int bi = wave; bi < nb; bi += kDrawThreads / 64) {
            const int64_t cb = (b0 + bi) * kBatch;
            const int qn = (int)(nch - cb < kBatch ? nch - cb : kBatch);
            const uint32_t v = rh[bi * 64 + lane];
            uint32_t res = 0;
            for (int wl = 0; wl < 6; wl += 3) {
                const uint32_t lo0 = __shfl(v, wl);
                const bool bad = __ballot(w == wl && q < qn && v != lo0) != 0u;
                uint32_t kk = (w == wl + 2 && q < qn) ? v : 0u;
                kk += __shfl_xor(kk, 8);
                kk += __shfl_xor(kk, 16);
                kk += __shfl_xor(kk, 32);
                const uint32_t ks = __shfl(kk, wl + 2);
                const bool ok = !bad && lo0 != 0xFFFFFFFFu && ks <= 0x7FFFFFu;
                if (lane == wl) res = ok ? lo0 : 0xFFFFFFFFu;
                if (lane == wl + 1) res = ok ? 0x7FFFFFu - ks : 0u;
                if (lane == wl + 2) res = ok ? ks : 0u;
            }
            if (lane < kHeadWords) ragg[bi * kHeadWords + lane] = res;
        }
        // the round's chunks on the likely-slow list, up to kStage of them
        for (int e0 = 0; e0 < n_list; e0 += kDrawThreads) {
            const int base_n = st_n;
            if (base_n >= kStage) break;
            const uint32_t id = e0 == 0 ? first_ids : (e0 + tid < n_list ? slow_list[e0 + tid] : 0xFFFFFFFFu);
            const bool f = e0 + tid < n_list && (int64_t)id >= c_lo && (int64_t)id < c_hi && (int64_t)id < nch;
            const uint64_t bal = __ballot(f);
            if (lane == 0) wcnt[wave] = __popcll(bal);
            __syncthreads();
            int before = base_n;
            for (int k = 0; k < wave; k++) before += wcnt[k];
            const int slot = before + __popcll(bal & ((1ull << lane) - 1ull));
            if (f && slot < kStage) st_id[slot] = (int)id;
            __syncthreads();
            if (tid == 0) {
                int tot = base_n;
                for (int k = 0; k < kDrawThreads / 64; k++) tot += wcnt[k];
                st_n = tot < kStage ? tot : kStage;
            }
            __syncthreads();
        }
        const int nst = st_n;
        {  // their terms (four per thread per load) and block ranges, loads all in flight
            constexpr int kPer = kStage * kDrawChunk / 4 / kDrawThreads;
            f32x4 v[kPer];
#pragma unroll
            for (int j = 0; j < kPer; j++) {
                const int k = j * kDrawThreads + tid;  // float4 index: slot k / 64, offset 4 * (k % 64)
                if (k < nst * (kDrawChunk / 4)) {
                    const int64_t i = (int64_t)st_id[k / (kDrawChunk / 4)] * kDrawChunk + 4 * (k % (kDrawChunk / 4));
                    v[j] = i + 4 <= n ? *reinterpret_cast<const f32x4 *>(terms + i)
                                      : f32x4{i < n ? terms[i] : 0.0f, i + 1 < n ? terms[i + 1] : 0.0f,
                                              i + 2 < n ? terms[i + 2] : 0.0f, 0.0f};
                }
            }
            uint32_t sk[kStage * kSubWords / kDrawThreads];
#pragma unroll
            for (int j = 0; j < kStage * kSubWords / kDrawThreads; j++) {
                const int k = j * kDrawThreads + tid;
                if (k < nst * kSubWords) sk[j] = subk[(int64_t)st_id[k / kSubWords] * kSubWords + k % kSubWords];
            }
#pragma unroll
            for (int j = 0; j < kPer; j++) {
                const int k = j * kDrawThreads + tid;
                if (k < nst * (kDrawChunk / 4)) reinterpret_cast<f32x4 *>(st_terms)[k] = v[j];
            }
#pragma unroll
            for (int j = 0; j < kStage * kSubWords / kDrawThreads; j++) {
                const int k = j * kDrawThreads + tid;
                if (k < nst * kSubWords) st_subk[k] = sk[j];
            }
        }
        __syncthreads();
        return nb;
    };

    // One chunk's or one batch's range tests on the header words base..base+5 of hv.
    auto range_step = [&](uint32_t &A, uint32_t hv, int base) -> bool {
        const uint32_t lo_a = __builtin_amdgcn_readlane(hv, base + 0);
        const uint32_t sp_a = __builtin_amdgcn_readlane(hv, base + 1);
        const uint32_t k_a = __builtin_amdgcn_readlane(hv, base + 2);
        const uint32_t lo_b = __builtin_amdgcn_readlane(hv, base + 3);
        const uint32_t sp_b = __builtin_amdgcn_readlane(hv, base + 4);
        const uint32_t k_b = __builtin_amdgcn_readlane(hv, base + 5);
        const bool ok_a = A - lo_a <= sp_a, ok_b = A - lo_b <= sp_b;
        A += ok_a ? k_a : (ok_b ? k_b : 0u);
        return ok_a || ok_b;
    };
    // One chunk from A (bits of the running sum at its start, wave-uniform) to its end: the
    // chunk's range tests; else runs of blocks, lane s holding block s: the longest run from
    // block s0 that one binade takes (an inclusive prefix sum of the blocks' increments and a
    // ballot of the first block whose range test fails; within a run every block's own test
    // holds, since A + prefix stays in the binade), else block s0's terms one per lane, added in
    // order through readlane. The block ranges come from LDS when the chunk is staged; stv holds
    // the staged chunk ids, one per lane.
    auto step = [&](uint32_t A, uint32_t hv, int q, int64_t c, int stv) -> uint32_t {
        A = __builtin_amdgcn_readfirstlane(A);  // wave-uniform: keep the walk on scalar registers
        if (range_step(A, hv, kHeadWords * q)) return A;
        const uint64_t hit = __ballot(stv == (int)c);
        const bool staged = hit != 0u;
        const int slot = staged ? __builtin_ctzll(hit) : 0;
        const uint32_t kv = lane < kSubWords ? (staged ? st_subk[slot * kSubWords + lane] : subk[c * kSubWords + lane]) : 0u;
        const float *rt = staged ? st_terms + slot * kDrawChunk : terms + c * kDrawChunk;
        const int64_t left = n - c * kDrawChunk;
        const int nbk = (int)(left >= kDrawChunk ? kDrawSubs : (left + kDrawSub - 1) / kDrawSub);
        const int bl = lane & (kDrawSubs - 1);
        uint32_t lo_x[2], k_x[2];
#pragma unroll
        for (int x = 0; x < 2; x++) {
            lo_x[x] = __shfl(kv, kBlockWords * bl + 3 * x);
            k_x[x] = __shfl(kv, kBlockWords * bl + 3 * x + 2);
        }
        const uint32_t ea = __builtin_amdgcn_readlane(hv, kHeadWords * q + 6);
        int s0 = 0;
        while (s0 < nbk) {
            bool moved = false;
#pragma unroll
            for (int x = 0; x < 2; x++) {
                const uint32_t lo = (ea + 127u + (uint32_t)x) << 23;  // every valid block's lo
                const uint32_t base = A - lo;
                if (moved || base > 0x7FFFFFu) continue;
                const bool in = lane >= s0 && lane < nbk;
                uint32_t P = in ? k_x[x] : 0u;
                P += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)P, 0x111, 0xF, 0xF, true);  // row_shr:1
                P += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)P, 0x112, 0xF, 0xF, true);  // row_shr:2
                P += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)P, 0x114, 0xF, 0xF, true);  // row_shr:4
                const bool ok = lo_x[x] == lo && P <= 0x7FFFFFu - base;  // K <= 2^23 - 1, so P < 2^26
                const uint64_t fail = __ballot(in && !ok);
                const int se = fail != 0u ? __builtin_ctzll(fail) : nbk;
                if (se > s0) {
                    A += __builtin_amdgcn_readlane(P, se - 1);
                    s0 = se;
                    moved = true;
                }
            }
            if (moved) continue;
            const int64_t sb = c * kDrawChunk + s0 * kDrawSub;
            const int m = (int)(n - sb < kDrawSub ? n - sb : kDrawSub);
            const int tb = __builtin_bit_cast(int, lane < m ? rt[s0 * kDrawSub + lane] : 0.0f);
            float a = __builtin_bit_cast(float, A);
            if (m == kDrawSub) {
#pragma unroll
                for (int j = 0; j < kDrawSub; j++) a += __builtin_bit_cast(float, __builtin_amdgcn_readlane(tb, j));
            } else {
                for (int j = 0; j < m; j++) a += __builtin_bit_cast(float, __builtin_amdgcn_readlane(tb, j));
            }
            A = __builtin_amdgcn_readfirstlane(__builtin_bit_cast(uint32_t, a));
            s0++;
        }
        return A;
    };

    uint32_t A = 0;  // bits of the running sum (wave 0)
    int mk = 0;      // marks of 64 batches gather in one VGPR of wave 0 (lane b % 64), stored together
    for (int64_t b0 = 0; b0 < nbat; b0 += kRoundBatches) {
        const int nb = stage_round(b0);
        if (wave == 0) {
            const int stv = lane < st_n ? st_id[lane] : -1;
            uint32_t nc = rh[lane], na = ragg[lane & (kHeadWords - 1)];
            for (int bi = 0; bi < nb; bi++) {
                const int64_t b = b0 + bi;
                const uint32_t cur = nc, ag = na;
                if (bi + 1 < nb) {  // the next batch's reads in flight during this one
                    nc = rh[(bi + 1) * 64 + lane];
                    na = ragg[(bi + 1) * kHeadWords + (lane & (kHeadWords - 1))];
                }
                mk = lane == (int)(b & 63) ? (int)A : mk;
                if ((b & 63) == 63 || b == nbat - 1) {
                    if (lane <= (int)(b & 63)) marks[(b & ~(int64_t)63) + lane] = (uint32_t)mk;
                }
                A = __builtin_amdgcn_readfirstlane(A);
                if (range_step(A, ag, 0)) continue;
                // chunk by chunk (not unrolled: one copy of the rarely used block path stays in the
                // instruction cache)
                const int qn = (int)(nch - b * kBatch < kBatch ? nch - b * kBatch : kBatch);
#pragma unroll 1
                for (int q = 0; q < qn; q++) A = step(A, cur, q, b * kBatch + q, stv);
            }
        }
        __syncthreads();
    }
    if (tid == 0) {
        marks[nbat] = A;
        sum_bits = A;
        if (MODE == kWalkSum) {
            hdr->sum = __builtin_bit_cast(float, A);
            hdr->kept = n;
        }
    }
    if (MODE == kWalkSum) return;
    __syncthreads();
    const float sum_e = __builtin_bit_cast(float, sum_bits);
    if (MODE == kWalkDraw && sum_e <= 0.0f) {  // sampler.mojo:295-296 (a NaN sum goes on to the walk, as there)
        if (tid == 0) {
            out[0] = order ? order[0] : 0;
            out[1] = 0;
        }
        return;
    }
    const float r = MODE == kWalkDraw ? target_arg * sum_e : target_arg;  // r = u * sum_e, or top_p
    // batches whose end sum is below r form a prefix (the sums never decrease); a NaN r counts
    // none and the walk below finds no index, as the reference's
    int64_t below = 0;
    for (int64_t k = tid; k < nbat; k += kDrawThreads) below += __builtin_bit_cast(float, marks[k + 1]) < r ? 1 : 0;
    for (int o = 32; o > 0; o >>= 1) below += __shfl_xor(below, o);
    if (lane == 0) cnt_s[wave] = below;
    __syncthreads();
    int64_t bb = 0;
    for (int k = 0; k < kDrawThreads / 64; k++) bb += cnt_s[k];
    // the batch's chunks again from its recorded start, up to the first whose end reaches r
    if (wave == 0) {
        int64_t jc = -1;
        uint32_t B = 0;
        if (bb < nbat) {
            B = marks[bb];
            const uint32_t cur = heads[bb * 64 + lane];
            for (int q = 0; q < kBatch; q++) {
                const int64_t c = bb * kBatch + q;
                if (c >= nch) break;
                const uint32_t E = step(B, cur, q, c, -1);
                if (r <= __builtin_bit_cast(float, E)) {
                    jc = c;
                    break;
                }
                B = E;
            }
        }
        if (tid == 0) {
            chunk_s = jc;
            start_bits = B;
        }
    }
    __syncthreads();
    const int64_t jc = chunk_s;
    int64_t pick = n - 1;
    if (jc >= 0) {  // that chunk's terms through LDS, re-added from its start in lane 0
        const int64_t i0 = jc * kDrawChunk;
        const int cnt = (int)(n - i0 < kDrawChunk ? n - i0 : kDrawChunk);
        if (tid < cnt) tile[tid] = terms[i0 + tid];
        __syncthreads();
        if (tid == 0) {
            int he;
            chain_tile<true>(tile, cnt, __builtin_bit_cast(float, start_bits), r, he);
            if (he >= 0) pick = i0 + he;
        }
    }
    if (tid == 0) {
        if (MODE == kWalkCut) {
            hdr->n = pick + 1;  // the cut index, n - 1 when there is none
        } else {
            out[0] = order ? order[pick] : pick;
            out[1] = 1;
        }
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
    DrawHdr *hdr = nullptr;    // candidate count after the truncations
    float *cmax = nullptr;     // per-chunk maxima of the candidates
    float *terms = nullptr;    // the final draw's exps
    double *csum = nullptr;    // per-chunk f64 sums of the exps
    uint32_t *heads = nullptr; // per-chunk headers (kHeadWords each), whole batches
    uint32_t *subk = nullptr;  // per-chunk block ranges (kSubWords each)
    uint32_t *slow_list = nullptr;  // chunks the records kernel lists as likely slow
    uint32_t *marks = nullptr; // bits of the running sum at the start of every batch of chunks, then the total
    int64_t *lists = nullptr;  // context tokens then suppress ids
    int64_t *lists_host = nullptr;       // pinned staging of the lists (hipHostMalloc), reused per call
    hipEvent_t lists_copied = nullptr;   // the last copy out of lists_host
    int64_t *result = nullptr;
    uint32_t *sel_hist = nullptr;  // top-k selection: 3 digit histograms of kSelBins
    uint32_t *sel_cnt = nullptr;   // per-workgroup counts below / equal to the threshold key
    uint64_t *sel_cand = nullptr;  // the selected (key, index) values, kSeqTile
    float *gpv = nullptr;      // the greedy branch's per-workgroup best values
    int64_t *gpi = nullptr;    // and their indices
    void *sort_tmp = nullptr;
    size_t sort_tmp_bytes = 0;
};

static void free_work(SamplerWork *w) {
    void *ps[] = {w->counts, w->mask,  w->vals,  w->keys,      w->keys_out, w->idx,   w->idx_out,
                  w->hdr,    w->cmax,  w->terms, w->csum,      w->heads,    w->subk,  w->slow_list,
                  w->marks,  w->lists, w->result, w->gpv,      w->gpi,      w->sort_tmp,
                  w->sel_hist, w->sel_cnt, w->sel_cand};
    for (void *p : ps)
        if (p) (void)hipFree(p);
    if (w->lists_host) (void)hipHostFree(w->lists_host);
    if (w->lists_copied) (void)hipEventDestroy(w->lists_copied);
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
        int64_t *old_lists = w->lists, *old_result = w->result, *old_host = w->lists_host;
        hipEvent_t old_event = w->lists_copied;
        w->lists = nullptr;
        w->lists_host = nullptr;
        w->lists_copied = nullptr;
        w->result = nullptr;
        free_work(w);
        w->lists = old_lists;
        w->lists_host = old_host;
        w->lists_copied = old_event;
        w->result = old_result;
        w->cap_ctx = keep_lists;
        AESIR_HIP_TRY(hipMalloc((void **)&w->counts, (size_t)V * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->mask, (size_t)V));
        AESIR_HIP_TRY(hipMalloc((void **)&w->vals, (size_t)V * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->keys, (size_t)V * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->keys_out, (size_t)V * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->idx, (size_t)V * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->idx_out, (size_t)V * 4));
        const int64_t nch = (V + kDrawChunk - 1) / kDrawChunk;
        AESIR_HIP_TRY(hipMalloc((void **)&w->hdr, sizeof(DrawHdr)));
        AESIR_HIP_TRY(hipMalloc((void **)&w->cmax, (size_t)nch * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->terms, (size_t)V * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->csum, (size_t)nch * 8));
        const int64_t nbat = (nch + kBatch - 1) / kBatch;
        AESIR_HIP_TRY(hipMalloc((void **)&w->heads, (size_t)nbat * 64 * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->subk, (size_t)nch * kSubWords * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->slow_list, (size_t)kSlowListMax * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->sel_hist, (size_t)3 * kSelBins * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->sel_cnt, (size_t)2 * ((V + kSelBlock - 1) / kSelBlock) * 4));
        AESIR_HIP_TRY(hipMalloc((void **)&w->sel_cand, (size_t)kSeqTile * 8));
        AESIR_HIP_TRY(hipMalloc((void **)&w->marks, (size_t)(nbat + 1) * 4));
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
        if (w->lists_host) (void)hipHostFree(w->lists_host);
        w->lists = nullptr;
        w->lists_host = nullptr;
        const int64_t cap = n_lists > 1024 ? n_lists : 1024;
        AESIR_HIP_TRY(hipMalloc((void **)&w->lists, (size_t)cap * 8));
        AESIR_HIP_TRY(hipHostMalloc((void **)&w->lists_host, (size_t)cap * 8, hipHostMallocDefault));
        w->cap_ctx = cap;
    }
    if (!w->lists_copied) AESIR_HIP_TRY(hipEventCreateWithFlags(&w->lists_copied, hipEventDisableTiming));
    if (!w->result) AESIR_HIP_TRY(hipMalloc((void **)&w->result, 16));
    if (!w->gpv) AESIR_HIP_TRY(hipMalloc((void **)&w->gpv, kGreedyParts * sizeof(float)));
    if (!w->gpi) AESIR_HIP_TRY(hipMalloc((void **)&w->gpi, kGreedyParts * sizeof(int64_t)));
    return AESIR_OK;
}

// The greedy branch's two launches: partial maxima of (at most) kGreedyParts workgroups, then one.
static int32_t launch_greedy(hipStream_t s, const h16 *logits, int64_t V, const uint8_t *mask, SamplerWork *w) {
    const int64_t want = (V + kGreedyThreads - 1) / kGreedyThreads;
    const int parts = (int)(want < kGreedyParts ? want : kGreedyParts);
    hipLaunchKernelGGL(sampler_greedy_part_kernel, dim3((unsigned)parts), dim3(kGreedyThreads), 0, s, logits, V, mask,
                       w->gpv, w->gpi);
    AESIR_LAUNCH_CHECK("sampler_greedy_part_kernel");
    hipLaunchKernelGGL(sampler_greedy_finish_kernel, dim3(1), dim3(kGreedyThreads), 0, s, w->gpv, w->gpi, parts,
                       w->result);
    AESIR_LAUNCH_CHECK("sampler_greedy_finish_kernel");
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
        AESIR_TRY(launch_greedy(s, (const h16 *)logits, vocab, nullptr, w));
        AESIR_HIP_TRY(hipMemcpyAsync(ctx->pinned_i64, w->result, 16, hipMemcpyDeviceToHost, s));
        AESIR_HIP_TRY(hipStreamSynchronize(s));
        *token = ctx->pinned_i64[0];
        return AESIR_OK;
    }
    if (n_lists > 0) {
        // through the pinned staging buffer (an asynchronous copy; a pageable source would be
        // staged synchronously by the runtime), once the previous call's copy out of it is done
        AESIR_HIP_TRY(hipEventSynchronize(w->lists_copied));
        if (n_context > 0) std::memcpy(w->lists_host, context, (size_t)n_context * 8);
        if (n_suppress > 0) std::memcpy(w->lists_host + n_context, suppress, (size_t)n_suppress * 8);
        AESIR_HIP_TRY(hipMemcpyAsync(w->lists, w->lists_host, (size_t)n_lists * 8, hipMemcpyHostToDevice, s));
        AESIR_HIP_TRY(hipEventRecord(w->lists_copied, s));
    }
    const unsigned g = (unsigned)((vocab + kSThreads - 1) / kSThreads < 4096 ? (vocab + kSThreads - 1) / kSThreads : 4096);
    hipLaunchKernelGGL(sampler_clear_kernel, dim3(g), dim3(kSThreads), 0, s, w->counts, w->mask, vocab, w->sel_hist,
                       3 * kSelBins);
    AESIR_LAUNCH_CHECK("sampler_clear_kernel");
    if (n_lists > 0) {
        const unsigned gl = (unsigned)((n_lists + kSThreads - 1) / kSThreads < 4096 ? (n_lists + kSThreads - 1) / kSThreads : 4096);
        hipLaunchKernelGGL(sampler_mark_kernel, dim3(gl), dim3(kSThreads), 0, s, w->lists, n_context,
                           w->lists + n_context, n_suppress, w->counts, w->mask, vocab);
        AESIR_LAUNCH_CHECK("sampler_mark_kernel");
    }
    uint64_t st = *rng_state;
    if (greedy) {
        AESIR_TRY(launch_greedy(s, (const h16 *)logits, vocab, w->mask, w));
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
        const bool select_k = k_on && cfg->top_k <= kSeqTile;
        if (select_k) {  // the first top_k of the stable sort, found without sorting the vocabulary
            const unsigned nb = (unsigned)((vocab + kSelBlock - 1) / kSelBlock);
            const uint32_t k = (uint32_t)cfg->top_k;
            hipLaunchKernelGGL(sampler_select_hist_kernel<0>, dim3(nb), dim3(kSThreads), 0, s, w->keys, vocab, w->sel_hist, k);
            hipLaunchKernelGGL(sampler_select_hist_kernel<1>, dim3(nb), dim3(kSThreads), 0, s, w->keys, vocab, w->sel_hist, k);
            hipLaunchKernelGGL(sampler_select_hist_kernel<2>, dim3(nb), dim3(kSThreads), 0, s, w->keys, vocab, w->sel_hist, k);
            AESIR_LAUNCH_CHECK("sampler_select_hist_kernel");
            hipLaunchKernelGGL(sampler_select_count_kernel, dim3(nb), dim3(kSThreads), 0, s, w->keys, vocab, w->sel_hist, k,
                               w->sel_cnt);
            AESIR_LAUNCH_CHECK("sampler_select_count_kernel");
            hipLaunchKernelGGL(sampler_select_compact_kernel, dim3(nb), dim3(kSThreads), 0, s, w->keys, vocab,
                               w->sel_hist, k, w->sel_cnt, w->sel_cand);
            AESIR_LAUNCH_CHECK("sampler_select_compact_kernel");
            hipLaunchKernelGGL(sampler_select_sort_kernel, dim3(1), dim3(kSelSortThreads), 0, s, w->sel_cand, (int)k,
                               w->idx_out);
            AESIR_LAUNCH_CHECK("sampler_select_sort_kernel");
        } else if (p.sort) {
            size_t bytes = w->sort_tmp_bytes;
            AESIR_HIP_TRY(rocprim::radix_sort_pairs(w->sort_tmp, bytes, w->keys, w->keys_out, w->idx, w->idx_out,
                                                    (unsigned)vocab, 0, 32, s));
        }
        const int32_t *order = p.sort ? (const int32_t *)w->idx_out : nullptr;
        if (select_k) {
            // at most one LDS tile of candidates: truncations and the draw in one workgroup
            hipLaunchKernelGGL(sampler_tail_kernel, dim3(1), dim3(kTailThreads), 0, s, w->vals, order, vocab, p,
                               w->result);
            AESIR_LAUNCH_CHECK("sampler_tail_kernel");
        } else {
            // the chunked stages over hdr->n candidates (chunks past the count exit at once): each
            // running sum is a terms pass, a records pass and a walk
            const unsigned nch = (unsigned)((vocab + kDrawChunk - 1) / kDrawChunk);
            auto running_sum = [&](auto terms_mode, auto walk_mode, float target) -> int32_t {
                constexpr int TM = decltype(terms_mode)::value, WM = decltype(walk_mode)::value;
                hipLaunchKernelGGL(sampler_terms_kernel<TM>, dim3(nch), dim3(kDrawThreads), 0, s, w->vals, order,
                                   w->hdr, w->cmax, w->terms, w->csum);
                AESIR_LAUNCH_CHECK("sampler_terms_kernel");
                hipLaunchKernelGGL(sampler_records_kernel, dim3(nch), dim3(kDrawThreads), 0, s, w->terms, w->csum,
                                   w->hdr, w->heads, w->subk, w->slow_list);
                AESIR_LAUNCH_CHECK("sampler_records_kernel");
                hipLaunchKernelGGL(sampler_draw_kernel<WM>, dim3(1), dim3(kDrawThreads), 0, s, w->terms, w->heads,
                                   w->subk, w->slow_list, w->hdr, order, target, w->marks, w->result);
                AESIR_LAUNCH_CHECK("sampler_draw_kernel");
                return AESIR_OK;
            };
            using std::integral_constant;
            hipLaunchKernelGGL(sampler_set_n_kernel, dim3(1), dim3(1), 0, s, w->hdr, k_on ? cfg->top_k : vocab);
            AESIR_LAUNCH_CHECK("sampler_set_n_kernel");
            if (p_on) {  // apply_top_p (:119-147): the sum of the exps, then the cut on the probabilities
                AESIR_TRY(running_sum(integral_constant<int, kTermsExp>{}, integral_constant<int, kWalkSum>{}, 0.0f));
                AESIR_TRY(running_sum(integral_constant<int, kTermsProb>{}, integral_constant<int, kWalkCut>{},
                                      cfg->top_p));
            }
            if (m_on) {  // apply_min_p (:166-194): the sum of the exps, then the threshold cut
                AESIR_TRY(running_sum(integral_constant<int, kTermsExp>{}, integral_constant<int, kWalkSum>{}, 0.0f));
                hipLaunchKernelGGL(sampler_minp_cut_kernel, dim3(nch), dim3(kDrawThreads), 0, s, w->vals, order,
                                   w->hdr, cfg->min_p);
                AESIR_LAUNCH_CHECK("sampler_minp_cut_kernel");
                hipLaunchKernelGGL(sampler_minp_finish_kernel, dim3(1), dim3(1), 0, s, w->hdr);
                AESIR_LAUNCH_CHECK("sampler_minp_finish_kernel");
            }
            // the final draw (:284-305)
            hipLaunchKernelGGL(sampler_chunk_max_kernel, dim3(nch), dim3(kDrawThreads), 0, s, w->vals, order, w->hdr,
                               w->cmax);
            AESIR_LAUNCH_CHECK("sampler_chunk_max_kernel");
            AESIR_TRY(running_sum(integral_constant<int, kTermsDraw>{}, integral_constant<int, kWalkDraw>{}, p.u));
        }
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
