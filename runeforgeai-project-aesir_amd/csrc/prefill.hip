// Batched prefill for gfx950: the prompt's positions go through each layer together, as M-row
// GEMMs on the matrix cores, instead of one forward_pass per position (the reference's
// _run_generation prefills by position, aesir.mojo:358-374; the result is the same KV cache and
// the same next token up to f32 summation order).
//
// MFMA GEMM  C[M][N] = A[M][K] . B[N][K]^T, f16 in, f32 accumulate (v_mfma_f32_16x16x32_f16).
//   A (activations) and B (weights) are both K-contiguous, so every MFMA operand fragment is one
//   16-byte row load: lane l holds row (l % 16) and k = 8 (l / 16) .. +7 of its 16 x 32 slice, the
//   same k order for A and B. A workgroup is 4 waves over 64 adjacent output columns (16 weight
//   rows per wave) and a 32-row M tile. Each 64-wide K chunk of A and of the workgroup's weight
//   rows is copied straight from memory into an LDS stage (buffer loads with the LDS destination,
//   no register staging, weight lines fetched whole), and every wave reads its fragments with
//   ds_read_b128. Each wave keeps 8 accumulator tiles (rows 16i + 4 (l / 16) + e, column l % 16
//   in lane l).
//   Small-N GEMMs also split K over grid.z to put enough weight bytes in flight; their f32
//   partials are summed in a fixed order by the epilogue kernel (deterministic, no atomics).
//   Chunks of more than 64 positions use the wide-tile kernel below (the whole chunk in one
//   128-row M tile, 8 waves, 128-wide K chunks) instead; this 32-row kernel serves shorter chunks.
//   At M = 128 the GEMM is HBM-bound (128 flop/byte against MI355X's 312 flop/byte ridge).
#include <cmath>
#include <vector>

#include "common.hpp"
#include "device.hpp"
#include "kernels.hpp"
#include "mfma_gemm.hpp"
#include "model.hpp"

namespace aesir {


// Rows of A per workgroup tile and the workgroup count the K splits aim for in this 4-wave kernel
// with 64-wide K chunks. Measured on MI355X (TinyLlama 128-token prefill, ms, when this kernel
// served every chunk): M tile 128 / 256 workgroups 2.39; 64 / 256 2.31; 64 / 512 2.23; 32 / 512
// 2.22; 32 / 1024 2.37. Smaller tiles re-read the weights from L2 (one HBM read) but copy less of
// A per workgroup and fit more workgroups per CU. (The 8-wave wide-tile kernel below, with
// 128-wide chunks, does better with the whole 128-row chunk in one tile; this kernel now serves
// chunks of 64 rows or fewer.)
constexpr int kGemmMT = 32;
constexpr int kGemmWgTarget = 512;
constexpr int kGemmMF = kGemmMT / 16;   // MFMA row fragments per wave
constexpr int kGemmAJ = kGemmMT / 8 / 4;  // A copy instructions per wave per chunk
constexpr int kGemmWaves = 4;
constexpr int kGemmNW = 16;   // output columns per wave
constexpr int kGemmNT = kGemmWaves * kGemmNW;
constexpr int kGemmThreads = kGemmWaves * kWave;


constexpr int kGemmKC = 64;  // k per chunk (two MFMA k-steps)

// grid (N / 64, ceil(M / 128), splits): a 4-wave workgroup owns 64 output columns (16 per wave)
// and a kGemmMT-row M tile. With one split the epilogue is applied here; otherwise split z writes its
// f32 partial to P[z][M][N] for gemm_reduce_kernel. Requires K % 64 == 0 and 16-byte aligned rows
// (checked by the launcher). Each 64-wide K chunk
// of A (kGemmMT rows x 128 B) and of the workgroup's 64 weight rows (64 x 128 B) is copied by
// buffer_load_dwordx4 ... lds straight into one of S LDS stages: a wave instruction moves 8 whole
// 128-byte row segments (lane l: row l / 8, 16-byte granule l % 8), so every weight line is
// fetched whole by one instruction, and nothing passes through registers. Granule p of row r
// holds k-granule p ^ ((r >> 1) & 7), which spreads the 16 rows of an MFMA fragment read over
// all LDS banks. S - 1 chunks are in flight ahead of the MFMAs; the waits are explicit vmcnt
// counts (each wave issues 6 copies per chunk) followed by a workgroup barrier.
constexpr int kDmaRowBytes = 128;                      // one chunk of one row
constexpr int kDmaStageA = kGemmMT * kDmaRowBytes;      // 4 KB
constexpr int kDmaStage = kDmaStageA + kGemmNT * kDmaRowBytes;  // + 8 KB of weights
// Q8_0 weights: a chunk of a weight row is 64 int8 quants (64 B) plus its two f16 block scales.
constexpr int kDmaQRowBytes = 64;
constexpr int kDmaStageQ = kDmaStageA + kGemmNT * kDmaQRowBytes + kGemmNT * 4;  // A + quants + scales
// LDS stages (S - 1 chunks in flight). Measured on MI355X, TinyLlama 128-token prefill with the
// 32-row tile (12 KB stages): 2 stages 1.88 ms, 3 stages 1.74, 4 1.76, 6 1.89.
constexpr int kDmaStages = 3;                  // f16 weights
constexpr int kDmaStagesQ = 2;  // Q8_0 weights: 2 stages 1.94-1.97 ms, 3 stages 1.98-1.99, 4 stages 2.01 (TinyLlama)

__device__ __forceinline__ int dma_swz(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int dma_swz_q(int row) { return (row >> 2) & 3; }  // 4 granules per quant row


// Q8: B is Q8_0 (int8 quants [N][K] + f16 block scales Bs [N][K / 32]). A chunk's 64 weight rows
// are 64-byte quant segments (one copy per wave: 16 rows x 4 granules, granule p of row r holding
// k-granule p ^ ((r >> 2) & 3)) plus the rows' two scales (one dword copy, wave 0). Each B
// fragment is dequantized from LDS as f16(q * d) (dequant_q8x4, gemm_q8_0's rounding), so the
// product equals the f16 GEMM with the dequantized weights. Wave 0 issues one more copy per chunk
// than the others, and its wait count says so.
template <int EPI, bool Q8>
__global__ __launch_bounds__(kGemmThreads) void gemm_mfma_kernel(const h16 *__restrict__ A, int64_t M, int64_t K,
                                                                const void *__restrict__ B, int64_t N,
                                                                h16 *__restrict__ C, int64_t ldc,
                                                                float *__restrict__ P, const h16 *__restrict__ Bs) {
    constexpr int S = Q8 ? kDmaStagesQ : kDmaStages;
    constexpr int kStage = Q8 ? kDmaStageQ : kDmaStage;
    // copies per wave per chunk: A rows, then f16 weight rows, or Q8_0 quant rows (+ the scale
    // dword copy, issued by wave 0 only)
    constexpr int kCopiesF16 = kGemmAJ + kGemmNT / 8 / kGemmWaves;
    constexpr int kCopiesQ8 = kGemmAJ + 1;
    extern __shared__ __align__(16) uint8_t lds[];  // S stages of kStage bytes
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t m0 = (int64_t)blockIdx.y * kGemmMT;
    const int64_t nb = (int64_t)blockIdx.x * kGemmNT;
    const int r = lane & 15, g = lane >> 4;
    const int64_t nkc = K / kGemmKC, splits = gridDim.z, z = blockIdx.z;
    const int64_t c0 = nkc * z / splits, c1 = nkc * (z + 1) / splits;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void *)A, 0, (int)(M * K * 2), kBufferDword3);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void *)B, 0, (int)(N * K * (Q8 ? 1 : 2)), kBufferDword3);
    const int64_t KB = K / 32;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)Bs, 0, Q8 ? (int)(N * KB * 2) : 0, kBufferDword3);
    // copy instruction j of this wave: A rows 8 kGemmAJ wave + 8 j + lane / 8 (j < kGemmAJ), weight rows
    // 16 wave + 8 j + lane / 8 (j < 2); the per-lane byte offset holds the row and granule, the
    // chunk's k offset goes in the uniform soffset
    const int drow = lane >> 3, dp = lane & 7;
    int aoff[kGemmAJ], boff[2];
#pragma unroll
    for (int j = 0; j < kGemmAJ; j++) {
        const int row = 8 * kGemmAJ * wave + 8 * j + drow;
        aoff[j] = (int)((m0 + row) * K * 2) + ((dp ^ dma_swz(row)) << 4);
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int row = 16 * wave + 8 * j + drow;
        boff[j] = (int)((nb + row) * K * 2) + ((dp ^ dma_swz(row)) << 4);
    }
    const int qrow = 16 * wave + (lane >> 2), qp = lane & 3;  // Q8: quant copy lane -> (row, granule)
    const int qoff = (int)((nb + qrow) * K) + ((qp ^ dma_swz_q(qrow)) << 4);
    const int soff = (int)((nb + lane) * KB * 2);              // Q8: scale copy lane -> row
    auto issue = [&](int64_t c, int stage) {
        c = c < c1 ? c : c1 - 1;  // past the range: re-read the last chunk into a free stage
        const int kb = (int)(c * kDmaRowBytes);
        uint8_t *sa = lds + stage * kStage;
#pragma unroll
        for (int j = 0; j < kGemmAJ; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void *)(sa + (8 * kGemmAJ * wave + 8 * j) * kDmaRowBytes), 16, aoff[j],
                kb, 0, 0);
        if (Q8) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (__attribute__((address_space(3))) void *)(sa + kDmaStageA + 16 * wave * kDmaQRowBytes), 16, qoff,
                (int)(c * kDmaQRowBytes), 0, 0);
            if (wave == 0)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rs, (__attribute__((address_space(3))) void *)(sa + kDmaStageA + kGemmNT * kDmaQRowBytes), 4, soff,
                    (int)(c * 4), 0, 0);
        } else {
#pragma unroll
            for (int j = 0; j < 2; j++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rb, (__attribute__((address_space(3))) void *)(sa + kDmaStageA + (16 * wave + 8 * j) * kDmaRowBytes),
                    16, boff[j], kb, 0, 0);
        }
    };

    f32x4 acc[kGemmMF];
#pragma unroll
    for (int i = 0; i < kGemmMF; i++) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (c0 < c1) {
#pragma unroll
        for (int j = 0; j < S - 1; j++) issue(c0 + j, j);
        const int brow = 16 * wave + r;
        for (int64_t c = c0; c < c1; c++) {
            const int t = (int)(c - c0);
            // this wave's copies of chunk c landed (S - 2 later chunks may still be in flight)
            if (!Q8)
                __builtin_amdgcn_s_waitcnt(vm_wait(kCopiesF16 * (S - 2)));
            else if (wave == 0)
                __builtin_amdgcn_s_waitcnt(vm_wait((kCopiesQ8 + 1) * (S - 2)));
            else
                __builtin_amdgcn_s_waitcnt(vm_wait(kCopiesQ8 * (S - 2)));
            __builtin_amdgcn_s_barrier();                                // ... and every wave's
            issue(c + S - 1, (t + S - 1) % S);  // into the stage chunk c - 1 used
            const uint8_t *sa = lds + (t % S) * kStage, *sb = sa + kDmaStageA;
            u32x4 bf[2], a[2][kGemmMF];  // every fragment of the chunk is requested before the first MFMA
            uint2 bq[2];
            h16 bd[2];
#pragma unroll
            for (int q = 0; q < 2; q++) {
                if (Q8) {  // k 32q + 8g .. +7: half g & 1 of granule 2q + g / 2
                    bq[q] = *reinterpret_cast<const uint2 *>(
                        sb + brow * kDmaQRowBytes + (((2 * q + (g >> 1)) ^ dma_swz_q(brow)) << 4) + 8 * (g & 1));
                    bd[q] = reinterpret_cast<const h16 *>(sb + kGemmNT * kDmaQRowBytes)[2 * brow + q];
                } else {
                    bf[q] = ld16(sb + brow * kDmaRowBytes + (((4 * q + g) ^ dma_swz(brow)) << 4));
                }
#pragma unroll
                for (int i = 0; i < kGemmMF; i++) {
                    const int row = 16 * i + r;
                    a[q][i] = ld16(sa + row * kDmaRowBytes + (((4 * q + g) ^ dma_swz(row)) << 4));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (Q8) {
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    unsigned w[4];
                    dequant_q8x4(bq[q].x, bd[q], w[0], w[1]);
                    dequant_q8x4(bq[q].y, bd[q], w[2], w[3]);
                    bf[q] = u32x4{w[0], w[1], w[2], w[3]};
                }
            }
#pragma unroll
            for (int q = 0; q < 2; q++)
#pragma unroll
                for (int i = 0; i < kGemmMF; i++) acc[i] = mfma16x16x32(a[q][i], bf[q], acc[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_waitcnt(vm_wait(0));  // no copy may land in LDS after the workgroup ends
    }

    const int64_t n = nb + 16 * wave + r;
#pragma unroll
    for (int i = 0; i < kGemmMF; i++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int64_t m = m0 + 16 * i + 4 * g + e;
            const float v = acc[i][e];
            if (splits == 1) {
                const float partner = dpp_f<kDppXor1>(v);  // lane r ^ 1 holds column n ^ 1
                gemm_epilogue<EPI>(C, ldc, M, N, m, n, v, partner);
            } else if (m < M && n < N) {
                P[(z * M + m) * N + n] = v;
            }
        }
    }
}

// Wide-tile kernel for M > 64 and K % 128 == 0: the whole 128-position chunk in one M tile,
// NT = 64 or 32 columns per workgroup of 8 waves (4 x 2, each 32 x NT / 2), or 48 columns (8 x 1,
// each 16 x 48: 235 workgroups instead of 176 for an 11264-row gate/up), 128-wide K chunks
// (four MFMA k-steps per chunk), 3 LDS stages of (128 + NT) 256-byte rows. Every copy
// instruction moves 4 whole 256-byte row chunks (lane l: row l / 16, granule l % 16), granule p
// of row r holding k-granule p ^ (r & 15), so the 16 rows of a fragment read hit distinct banks.
// Every weight row is copied once (the 32 x 64 kernel copies it once per 32 rows) and each
// barrier covers 3 - 4 times the bytes. K splits over grid.z write f32 partials like the 32 x 64
// kernel's, for the same reduce and row kernels.
// Measured on MI355X (M = 128, weights cold, us; against the split 32 x 64 kernel):
//   11264 x 2048 (gate/up)  17.3 against 22.5   28672 x 4096  64 against 134
//   2560 x 2048 (QKV)       10.3 against 11.8    6144 x 4096  21.3 against 27.1
//   2048 x 2048 (O)          9.5 against  9.6    4096 x 4096  15.3 against 19.3
//   2048 x 5632 (down)      13.8 against 15.9    4096 x 14336 34.1 against 56.5
// (hipBLASLt's pick for 11264 x 2048, MT64x128x128: 18.9.) In the TinyLlama prefill the gate/up
// launch takes 21.6 us with 64 columns (176 workgroups) and 20.2 with 48 (235); 48-column QKV
// tiles (54 x 4 splits instead of 80 x 2) were slower with their reduce (12.9 against 12.5 us).
// waves along M and N of an NT-column tile
__host__ __device__ constexpr int wide_wm(int nt) { return nt == 48 ? 8 : 4; }
__host__ __device__ constexpr int wide_wn(int nt) { return nt == 48 ? 1 : 2; }
constexpr int kWideRB = kWideKC * 2;  // bytes of one row chunk
constexpr int kWideMaxSplits = 8;     // fused row kernels take up to 8 split partials
constexpr int kWideWgTarget = 256;    // the split count doubles while tiles x splits stays within this

// Q8_0 weights (q8): a chunk's weight rows are 128-byte quant segments (8 rows per copy
// instruction: lane l row l / 8, granule l % 8, granule p of row r holding k-granule p ^ ((r >> 1)
// & 7)) plus the rows' four f16 block scales (4-byte copies, two lanes per row); every B fragment
// is dequantized to f16(q * d) by dequant_q8x4, as in the 32 x 64 kernel.
__host__ __device__ constexpr int wide_stage_bytes(int nt, bool q8) {
    return q8 ? kWideMT * kWideRB + nt * kWideKC + nt * 8 : (kWideMT + nt) * kWideRB;
}
__device__ __forceinline__ int wide_qswz(int row) { return (row >> 1) & 7; }

template <int EPI, int NT, bool Q8>
__device__ __forceinline__ void gemm_wide_body(const h16 *__restrict__ A, int64_t M, int64_t K,
                                               const void *__restrict__ B, int64_t N, h16 *__restrict__ C,
                                               int64_t ldc, float *__restrict__ P, const h16 *__restrict__ Bs) {
    constexpr int kWideWM = wide_wm(NT), kWideWN = wide_wn(NT);
    constexpr int kW = kWideWM * kWideWN;
    static_assert(kW * kWave == kWideThreads, "8 waves");
    constexpr int kStage = wide_stage_bytes(NT, Q8);
    // f16: (128 + NT) / 4 copies of four 256-byte rows; waves below kExtra issue one more than
    // kCopies (NT = 48: 44 copies, 6 for waves 0-3 and 5 for waves 4-7)
    constexpr int kCopies = (kWideMT + NT) / 4 / kW, kExtra = (kWideMT + NT) / 4 % kW;
    static_assert((kWideMT + NT) % 4 == 0 && (!Q8 || kExtra == 0), "whole copy instructions");
    // Q8_0: 128 / 4 A copies (4 per wave), NT / 8 quant copies (waves 0 .. NT / 8 - 1) and NT / 32
    // scale copies (waves (NT / 8 + s) % 8)
    constexpr int kAq = kWideMT / 4 / kW, kQq = NT / 8, kSq = NT / 32;
    static_assert(kAq * 4 * kW == kWideMT && kQq <= kW && kSq <= kW, "Q8_0 copy plan");
    constexpr int MF = kWideMT / kWideWM / 16, NF = NT / kWideWN / 16, KQ = kWideKC / 32;
    extern __shared__ __align__(16) uint8_t lds[];  // kWideS stages of kStage bytes
    // wave index as a scalar, so that each copy's operand choice is a scalar select
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / kWideWN, wn = wave % kWideWN;
    const int64_t m0 = (int64_t)blockIdx.y * kWideMT, n0 = (int64_t)blockIdx.x * NT;
    const int r = lane & 15, g = lane >> 4;
    const int64_t nkc = K / kWideKC, splits = gridDim.z, z = blockIdx.z;
    const int64_t c0 = nkc * z / splits, c1 = nkc * (z + 1) / splits;
    const int64_t KB = K / 32;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void *)A, 0, (int)(M * K * 2), kBufferDword3);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void *)B, 0, (int)(N * K * (Q8 ? 1 : 2)), kBufferDword3);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)Bs, 0, Q8 ? (int)(N * KB * 2) : 0, kBufferDword3);
    // f16 copy j of this wave: stage rows 4 (kCopies wave + j) .. + 3 (A rows first, then weights);
    // Q8_0: A copy j rows 4 (kAq wave + j) .. + 3
    constexpr int kAC = Q8 ? kAq : kCopies + (kExtra ? 1 : 0);
    const int first = Q8 ? kAq * wave : kCopies * wave + (wave < kExtra ? wave : kExtra);  // first copy
    const bool extra = kExtra && wave < kExtra;  // wave-uniform: issues copy kAC - 1 too
    int off[kAC], ldsrow[kAC];
    bool isa[kAC];
#pragma unroll
    for (int j = 0; j < kAC; j++) {
        const int row0 = 4 * (first + j), row = row0 + (lane >> 4);
        isa[j] = row0 < kWideMT;
        ldsrow[j] = row0;
        const int64_t grow = isa[j] ? m0 + row : n0 + row - kWideMT;
        off[j] = (int)(grow * K * 2) + (((lane & 15) ^ (row & 15)) << 4);
    }
    const bool has_q = Q8 && wave < kQq;  // this wave's quant copy: rows 8 wave + lane / 8
    const int qrow = 8 * wave + (lane >> 3);
    const int qoff = (int)((n0 + qrow) * K) + (((lane & 7) ^ wide_qswz(qrow)) << 4);
    const int sidx = (wave - kQq + kW) % kW;  // this wave's scale copy (if sidx < kSq): rows 32 sidx + lane / 2
    const bool has_s = Q8 && sidx < kSq;
    const int soff = (int)((n0 + 32 * sidx + (lane >> 1)) * KB * 2) + 4 * (lane & 1);
    const int ncopy = Q8 ? kAq + (has_q ? 1 : 0) + (has_s ? 1 : 0) : kCopies;  // wave-uniform
    auto issue = [&](int64_t c, int stage) {
        c = c < c1 ? c : c1 - 1;  // past the split's end: re-read its last chunk into a free stage
        uint8_t *sa = lds + stage * kStage;
#pragma unroll
        for (int j = 0; j < kAC; j++)
            if (!kExtra || j < kCopies || extra)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(isa[j] ? ra : rb,
                                                     (__attribute__((address_space(3))) void *)(sa + ldsrow[j] * kWideRB),
                                                     16, off[j], (int)(c * kWideRB), 0, 0);
        if (Q8) {
            uint8_t *sq = sa + kWideMT * kWideRB;
            if (has_q)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rb, (__attribute__((address_space(3))) void *)(sq + 8 * wave * kWideKC), 16, qoff,
                    (int)(c * kWideKC), 0, 0);
            if (has_s)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rs, (__attribute__((address_space(3))) void *)(sq + NT * kWideKC + 32 * sidx * 8), 4, soff,
                    (int)(c * 8), 0, 0);
        }
    };
    // wait until only the copies of the next chunk are in flight (wave-uniform count)
    auto wait_chunk = [&]() {
        if (kExtra && !extra) __builtin_amdgcn_s_waitcnt(vm_wait(kCopies * (kWideS - 2)));
        else if (!Q8 || ncopy == kAq) __builtin_amdgcn_s_waitcnt(vm_wait(kAC * (kWideS - 2)));
        else if (ncopy == kAq + 1) __builtin_amdgcn_s_waitcnt(vm_wait((kAq + 1) * (kWideS - 2)));
        else __builtin_amdgcn_s_waitcnt(vm_wait((kAq + 2) * (kWideS - 2)));
    };
    f32x4 acc[MF][NF];
#pragma unroll
    for (int i = 0; i < MF; i++)
#pragma unroll
        for (int j = 0; j < NF; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < kWideS - 1; j++) issue(c0 + j, j);
    for (int64_t c = c0; c < c1; c++) {
        const int t = (int)((c - c0) % kWideS);
        wait_chunk();                                      // this wave's copies of chunk c ...
        __builtin_amdgcn_s_barrier();                      // ... and every wave's
        issue(c + kWideS - 1, (t + kWideS - 1) % kWideS);  // into the stage chunk c - 1 used
        const uint8_t *sa = lds + t * kStage, *sb = sa + kWideMT * kWideRB;
        u32x4 a[KQ][MF], b[KQ][NF];
        uint2 bq[KQ][NF];
        h16 bd[KQ][NF];
#pragma unroll
        for (int q = 0; q < KQ; q++) {
#pragma unroll
            for (int i = 0; i < MF; i++) {
                const int row = wm * (kWideMT / kWideWM) + 16 * i + r;
                a[q][i] = ld16(sa + row * kWideRB + (((4 * q + g) ^ (row & 15)) << 4));
            }
#pragma unroll
            for (int j = 0; j < NF; j++) {
                const int row = wn * (NT / kWideWN) + 16 * j + r;
                if (Q8) {  // k 32 q + 8 g .. + 7: half g & 1 of granule 2 q + g / 2; block q of the chunk
                    bq[q][j] = *reinterpret_cast<const uint2 *>(sb + row * kWideKC +
                                                                (((2 * q + (g >> 1)) ^ wide_qswz(row)) << 4) + 8 * (g & 1));
                    bd[q][j] = reinterpret_cast<const h16 *>(sb + NT * kWideKC + row * 8)[q];
                } else {
                    b[q][j] = ld16(sb + row * kWideRB + (((4 * q + g) ^ ((row + kWideMT) & 15)) << 4));
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (Q8) {
#pragma unroll
            for (int q = 0; q < KQ; q++)
#pragma unroll
                for (int j = 0; j < NF; j++) {
                    unsigned w[4];
                    dequant_q8x4(bq[q][j].x, bd[q][j], w[0], w[1]);
                    dequant_q8x4(bq[q][j].y, bd[q][j], w[2], w[3]);
                    b[q][j] = u32x4{w[0], w[1], w[2], w[3]};
                }
        }
#pragma unroll
        for (int q = 0; q < KQ; q++)
#pragma unroll
            for (int i = 0; i < MF; i++)
#pragma unroll
                for (int j = 0; j < NF; j++) acc[i][j] = mfma16x16x32(a[q][i], b[q][j], acc[i][j]);
        __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(0));  // no copy may land in LDS after the workgroup ends
#pragma unroll
    for (int i = 0; i < MF; i++)
#pragma unroll
        for (int j = 0; j < NF; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int64_t m = m0 + wm * (kWideMT / kWideWM) + 16 * i + 4 * g + e;
                const int64_t n = n0 + wn * (NT / kWideWN) + 16 * j + r;
                const float v = acc[i][j][e];
                if (splits == 1) {
                    const float partner = dpp_f<kDppXor1>(v);  // lane r ^ 1 holds column n ^ 1
                    gemm_epilogue<EPI>(C, ldc, M, N, m, n, v, partner);
                } else if (m < M && n < N) {
                    P[(z * M + m) * N + n] = v;
                }
            }
}

// One kernel per (epilogue, tile width, weight type); the template body above is shared.
#define AESIR_WIDE_KERNEL(EPIV, NTV, Q8V, SUF)                                                                   \
    __global__ __launch_bounds__(kWideThreads) void gemm_wide_kernel_##EPIV##_##NTV##SUF(                       \
        const h16 *__restrict__ A, int64_t M, int64_t K, const void *__restrict__ B, int64_t N, h16 *__restrict__ C, \
        int64_t ldc, float *__restrict__ P, const h16 *__restrict__ Bs) {                                         \
        gemm_wide_body<EPIV, NTV, Q8V>(A, M, K, B, N, C, ldc, P, Bs);                                           \
    }
AESIR_WIDE_KERNEL(0, 64, false, )
AESIR_WIDE_KERNEL(0, 32, false, )
AESIR_WIDE_KERNEL(1, 64, false, )
AESIR_WIDE_KERNEL(1, 32, false, )
AESIR_WIDE_KERNEL(2, 64, false, )
AESIR_WIDE_KERNEL(2, 32, false, )
AESIR_WIDE_KERNEL(0, 48, false, )
AESIR_WIDE_KERNEL(1, 48, false, )
AESIR_WIDE_KERNEL(2, 48, false, )
AESIR_WIDE_KERNEL(0, 64, true, _q8)
AESIR_WIDE_KERNEL(0, 32, true, _q8)
AESIR_WIDE_KERNEL(1, 64, true, _q8)
AESIR_WIDE_KERNEL(1, 32, true, _q8)
AESIR_WIDE_KERNEL(2, 64, true, _q8)
AESIR_WIDE_KERNEL(2, 32, true, _q8)
#undef AESIR_WIDE_KERNEL

typedef void (*WideKernelFn)(const h16 *, int64_t, int64_t, const void *, int64_t, h16 *, int64_t, float *,
                             const h16 *);
template <int EPI, int NT, bool Q8>
static WideKernelFn wide_kernel() {
    if constexpr (Q8) {
        if constexpr (EPI == kEpiStore) return NT == 64 ? gemm_wide_kernel_0_64_q8 : gemm_wide_kernel_0_32_q8;
        else if constexpr (EPI == kEpiResidual) return NT == 64 ? gemm_wide_kernel_1_64_q8 : gemm_wide_kernel_1_32_q8;
        else return NT == 64 ? gemm_wide_kernel_2_64_q8 : gemm_wide_kernel_2_32_q8;
    } else if constexpr (NT == 48) {
        if constexpr (EPI == kEpiStore) return gemm_wide_kernel_0_48;
        else if constexpr (EPI == kEpiResidual) return gemm_wide_kernel_1_48;
        else return gemm_wide_kernel_2_48;
    } else {
        if constexpr (EPI == kEpiStore) return NT == 64 ? gemm_wide_kernel_0_64 : gemm_wide_kernel_0_32;
        else if constexpr (EPI == kEpiResidual) return NT == 64 ? gemm_wide_kernel_1_64 : gemm_wide_kernel_1_32;
        else return NT == 64 ? gemm_wide_kernel_2_64 : gemm_wide_kernel_2_32;
    }
}

// Tile width and K splits of the wide-tile kernel, or nt = 0 when the 32 x 64 kernel serves the
// GEMM (M <= 64, K % 128 != 0, or a 32-bit byte range exceeded). NT = 64 from 4096 columns up, 32
// below; the split count doubles while it divides the K chunks evenly, leaves at least 4 chunks per
// split and keeps tiles x splits within kWideWgTarget.
struct WidePlan {
    int nt;
    int64_t splits;
};
static WidePlan wide_plan_nt(int64_t M, int64_t K, int64_t N, int nt) {
    const int64_t tiles = ((N + nt - 1) / nt) * ((M + kWideMT - 1) / kWideMT), nkc = K / kWideKC;
    int64_t s = 1;
    while (2 * s <= kWideMaxSplits && tiles * 2 * s <= kWideWgTarget && nkc % (2 * s) == 0 && nkc / (2 * s) >= 4) s *= 2;
    return {nt, s};
}
static int64_t wide_workgroups(int64_t M, int64_t N, const WidePlan &p) {
    return ((N + p.nt - 1) / p.nt) * ((M + kWideMT - 1) / kWideMT) * p.splits;
}
static WidePlan wide_plan(int64_t M, int64_t K, int64_t N, bool q8 = false) {
    const int64_t lim = (int64_t)1 << 31;
    if (M <= 64 || K % kWideKC != 0 || (M + kWideMT) * K * 2 >= lim || (N + 64) * K * 2 >= lim) return {0, 1};
    const WidePlan p = wide_plan_nt(M, K, N, N >= 4096 ? 64 : 32);
    if (q8 || p.nt != 64) return p;
    // 48-column tiles (f16 weights) where 64-column ones leave part of the chip idle and 48 fill
    // more of it in one pass
    const WidePlan p48 = wide_plan_nt(M, K, N, 48);
    const int64_t w64 = wide_workgroups(M, N, p), w48 = wide_workgroups(M, N, p48);
    return w64 < kWideWgTarget && w48 > w64 && w48 <= kWideWgTarget ? p48 : p;
}

template <int EPI, int NT, bool Q8>
static int32_t launch_wide(hipStream_t s, const void *A, int64_t M, int64_t K, const void *B, int64_t N, void *C,
                           int64_t ldc, float *part, int64_t splits, const void *Bs) {
    static std::atomic<uint64_t> lds_set{0};
    constexpr int lds = kWideS * wide_stage_bytes(NT, Q8);
    AESIR_TRY(raise_lds_limit(reinterpret_cast<const void *>(wide_kernel<EPI, NT, Q8>()), lds, lds_set));
    const dim3 grid((unsigned)((N + NT - 1) / NT), (unsigned)((M + kWideMT - 1) / kWideMT), (unsigned)splits);
    hipLaunchKernelGGL((wide_kernel<EPI, NT, Q8>()), grid, dim3(kWideThreads), lds, s, (const h16 *)A, M, K, B, N,
                       (h16 *)C, ldc, part, (const h16 *)Bs);
    return AESIR_OK;
}

// Sums the split partials of each output in split order and applies the epilogue; one thread
// per output, consecutive threads on consecutive columns (pairs of SwiGLU columns are adjacent).
template <int EPI>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const float *__restrict__ P, int64_t splits, int64_t M,
                                                          int64_t N, h16 *__restrict__ C, int64_t ldc) {
    const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = M * N;
    const int64_t oc = o < total ? o : total - 1;  // tail threads repeat the last output, store nothing
    float v = 0.0f;
    for (int64_t z = 0; z < splits; z++) v += P[z * total + oc];
    const float partner = dpp_f<kDppXor1>(v);  // N even for SwiGLU: o ^ 1 is column n ^ 1
    if (o < total) gemm_epilogue<EPI>(C, ldc, M, N, oc / N, oc % N, v, partner);
}

// The kernel addresses each operand through a buffer resource with a 32-bit byte range.
static bool mfma_shape_ok(const void *A, int64_t M, int64_t K, const void *B, int64_t N) {
    const int64_t lim = (int64_t)1 << 31;  // (Q8_0 quant rows are half as long: the f16 bound covers them)
    return K % 64 == 0 && ((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0 && (M + kGemmMT) * K * 2 < lim &&
           (N + kGemmNT) * K * 2 < lim;
}

// K splits for a GEMM: enough workgroups to keep the chip's memory pipes full (about
// kGemmWgTarget) while every split keeps at least 8 k-steps.
static int64_t gemm_splits(int64_t M, int64_t K, int64_t N) {
    const int64_t tiles = ((N + kGemmNT - 1) / kGemmNT) * ((M + kGemmMT - 1) / kGemmMT);
    int64_t s = (kGemmWgTarget + tiles - 1) / tiles;
    const int64_t max_s = K / 256;  // at least four 64-wide chunks per split
    if (s > max_s) s = max_s;
    return s < 1 ? 1 : s;
}

// The shape half of prefill_mfma_ok: true when a model of this shape runs every prefill GEMM on
// the matrix cores (its arena buffers and weights are 256-byte aligned, which covers the rest), so
// the f16 gate/up products of the fallback need no buffer.
bool prefill_gemm_shapes_ok(int64_t rows, int64_t dim, int64_t qkv_n, int64_t ffn) {
    const int64_t lim = (int64_t)1 << 31;
    const int64_t shapes[4][2] = {{dim, qkv_n}, {dim, dim}, {dim, 2 * ffn}, {ffn, dim}};  // (K, N)
    for (auto &kn : shapes)
        if (kn[0] % 64 != 0 || (rows + kGemmMT) * kn[0] * 2 >= lim || (kn[1] + kGemmNT) * kn[0] * 2 >= lim) return false;
    return true;
}

int64_t prefill_part_floats(int64_t rows, int64_t dim, int64_t qkv_n, int64_t ffn) {
    const int64_t shapes[4][2] = {{dim, qkv_n}, {dim, dim}, {dim, 2 * ffn}, {ffn, dim}};  // (K, N)
    int64_t most = 0;
    // every chunk length up to `rows` (a shorter chunk may plan more K splits)
    for (int64_t m = 1; m <= rows; m++)
        for (auto &kn : shapes) {
            if (kn[0] % 64 != 0) continue;
            for (bool q8 : {false, true}) {
                const WidePlan wp = wide_plan(m, kn[0], kn[1], q8);
                const int64_t sp = wp.nt ? wp.splits : gemm_splits(m, kn[0], kn[1]);
                if (sp > 1 && sp * m * kn[1] > most) most = sp * m * kn[1];
            }
        }
    return most;
}

// With `defer` set, a split GEMM leaves its f32 partials in `part` for a fused row kernel of the
// caller instead of launching gemm_reduce_kernel; *splits_out receives the split count.
// Bs non-null: B is Q8_0 quants with these f16 block scales.
template <int EPI>
static int32_t launch_mfma(hipStream_t s, const void *A, int64_t M, int64_t K, const void *B, int64_t N, void *C,
                           int64_t ldc, float *part, int64_t part_floats, const char *name, bool defer = false,
                           int64_t *splits_out = nullptr, const void *Bs = nullptr) {
    const int64_t gx = (N + kGemmNT - 1) / kGemmNT, gy = (M + kGemmMT - 1) / kGemmMT;
    if (gx > 2147483647 || gy > 65535) return fail(AESIR_ERR_UNSUPPORTED, "%s: GEMM grid too large", name);
    if (EPI == kEpiSwiglu && (N & 1)) return fail(AESIR_ERR_INVALID, "%s: odd gate/up column count", name);
    if (const WidePlan wp = wide_plan(M, K, N, Bs != nullptr); wp.nt) {
        int64_t splits = wp.splits;
        while (splits > 1 && splits * M * N > part_floats) splits /= 2;
        if (wp.nt == 48)
            AESIR_TRY((launch_wide<EPI, 48, false>(s, A, M, K, B, N, C, ldc, part, splits, nullptr)));
        else if (wp.nt == 64 && Bs)
            AESIR_TRY((launch_wide<EPI, 64, true>(s, A, M, K, B, N, C, ldc, part, splits, Bs)));
        else if (Bs)
            AESIR_TRY((launch_wide<EPI, 32, true>(s, A, M, K, B, N, C, ldc, part, splits, Bs)));
        else if (wp.nt == 64)
            AESIR_TRY((launch_wide<EPI, 64, false>(s, A, M, K, B, N, C, ldc, part, splits, nullptr)));
        else
            AESIR_TRY((launch_wide<EPI, 32, false>(s, A, M, K, B, N, C, ldc, part, splits, nullptr)));
        AESIR_LAUNCH_CHECK(name);
        if (splits_out) *splits_out = splits;
        if (splits > 1 && !defer) {
            const int64_t blocks = (M * N + 255) / 256;
            hipLaunchKernelGGL(gemm_reduce_kernel<EPI>, dim3((unsigned)blocks), dim3(256), 0, s, (const float *)part,
                               splits, M, N, (h16 *)C, ldc);
            AESIR_LAUNCH_CHECK("gemm_reduce_kernel");
        }
        return AESIR_OK;
    }
    int64_t splits = gemm_splits(M, K, N);
    while (splits > 1 && splits * M * N > part_floats) splits--;
    const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)splits);
    if (Bs)
        hipLaunchKernelGGL((gemm_mfma_kernel<EPI, true>), grid, dim3(kGemmThreads), kDmaStagesQ * kDmaStageQ, s,
                           (const h16 *)A, M, K, B, N, (h16 *)C, ldc, part, (const h16 *)Bs);
    else
        hipLaunchKernelGGL((gemm_mfma_kernel<EPI, false>), grid, dim3(kGemmThreads), kDmaStages * kDmaStage, s,
                           (const h16 *)A, M, K, B, N, (h16 *)C, ldc, part, (const h16 *)nullptr);
    AESIR_LAUNCH_CHECK(name);
    if (splits_out) *splits_out = splits;
    if (splits > 1 && !defer) {
        const int64_t blocks = (M * N + 255) / 256;
        hipLaunchKernelGGL(gemm_reduce_kernel<EPI>, dim3((unsigned)blocks), dim3(256), 0, s, (const float *)part, splits,
                           M, N, (h16 *)C, ldc);
        AESIR_LAUNCH_CHECK("gemm_reduce_kernel");
    }
    return AESIR_OK;
}

static int32_t launch_swiglu_pairs(hipStream_t s, const void *gu, void *act, int64_t n);

// Q8_0 planes (int8 quants [N][K], f16 block scales [N][K / 32]) -> f16 [N][K] with
// w = f16(f16(q) d) per weight (dequant_q8x4: the rounding of gemm_q8_0, compute.mojo:1062-1063,
// and of every Q8_0 kernel here). K % 32 == 0; each thread converts 16 weights of one block.
__global__ __launch_bounds__(256) void q8_dequant_rows_kernel(const int8_t *__restrict__ q, const h16 *__restrict__ d,
                                                              int64_t N, int64_t K, h16 *__restrict__ out) {
    const int64_t total = N * K / 16;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t e = i * 16, n = e / K, k = e % K;
        const u32x4 qv = ld16(q + e);
        const h16 dd = d[n * (K / 32) + k / 32];
        unsigned w[8];
        dequant_q8x4(qv.x, dd, w[0], w[1]);
        dequant_q8x4(qv.y, dd, w[2], w[3]);
        dequant_q8x4(qv.z, dd, w[4], w[5]);
        dequant_q8x4(qv.w, dd, w[6], w[7]);
        st16(out + e, u32x4{w[0], w[1], w[2], w[3]});
        st16(out + e + 8, u32x4{w[4], w[5], w[6], w[7]});
    }
}

static int32_t launch_q8_dequant_rows(hipStream_t s, const void *q, const void *d, int64_t N, int64_t K, void *out) {
    if (K % 32 != 0 || ((uintptr_t)q & 15) || ((uintptr_t)out & 15))
        return fail(AESIR_ERR_UNSUPPORTED, "q8_dequant_rows: K %% 32 and 16-byte aligned rows required");
    int64_t g = (N * K / 16 + 255) / 256;
    if (g > 16384) g = 16384;
    hipLaunchKernelGGL(q8_dequant_rows_kernel, dim3((unsigned)g), dim3(256), 0, s, (const int8_t *)q, (const h16 *)d, N,
                       K, (h16 *)out);
    AESIR_LAUNCH_CHECK("q8_dequant_rows_kernel");
    return AESIR_OK;
}

// F16 GEMMs of chunks of at least this many rows run on hipBLASLt (blas.hip): from here on the
// library tile is faster than the wide-tile kernel plus the row kernel the library path needs for
// its epilogue. Measured on MI355X, TinyLlama shapes, 1024 rows (µs per GEMM, library / wide tile):
// QKV 16 / 33, gate/up 36 / 104, down 30 / 57.
constexpr int64_t kBlasMinRows = 256;
constexpr int64_t kBlasWorkspace = 32 << 20;

// The library path of prefill_gemm: the plain product in f16 (store; gate/up pairs, then the SwiGLU
// row kernel) or in f32 (residual: one partial for the caller's fused residual + norm row kernel,
// or gemm_reduce_kernel when not deferred), so every rounding is the epilogue's own.
// AESIR_ERR_UNSUPPORTED when the library has no algorithm (the caller takes its own kernel).
template <int EPI>
static int32_t prefill_gemm_blas(aesir_model *m, hipStream_t s, const void *W, const void *A, int64_t M, int64_t K,
                                 int64_t N, void *C, int64_t ldc, bool defer, int64_t *splits_out, const float **part_out) {
    aesir_ctx *ctx = m->ctx;
    if (EPI == kEpiStore) {
        if (ldc != N) return AESIR_ERR_UNSUPPORTED;
        AESIR_TRY(blas_gemm_nt(ctx, s, A, M, K, W, N, C, false, m->pf_blas_ws, kBlasWorkspace));
    } else if (EPI == kEpiSwiglu) {
        if (ldc != N / 2) return AESIR_ERR_UNSUPPORTED;
        AESIR_TRY(blas_gemm_nt(ctx, s, A, M, K, W, N, m->pf_gu, false, m->pf_blas_ws, kBlasWorkspace));
        AESIR_TRY(launch_swiglu_pairs(s, m->pf_gu, C, M * (N / 2)));
    } else {
        const float *part = (const float *)m->pf_gu;
        AESIR_TRY(blas_gemm_nt(ctx, s, A, M, K, W, N, m->pf_gu, true, m->pf_blas_ws, kBlasWorkspace));
        if (defer) {
            if (splits_out) *splits_out = 1;
            if (part_out) *part_out = part;
            return AESIR_OK;
        }
        const int64_t blocks = (M * N + 255) / 256;
        hipLaunchKernelGGL(gemm_reduce_kernel<EPI>, dim3((unsigned)blocks), dim3(256), 0, s, part, (int64_t)1, M, N,
                           (h16 *)C, ldc);
        AESIR_LAUNCH_CHECK("gemm_reduce_kernel");
    }
    if (splits_out) *splits_out = 1;
    if (part_out) *part_out = nullptr;
    return AESIR_OK;
}

// A GEMM of the prefill on the model's matrix w (rows N, K wide): F16 weights in chunks of
// kBlasMinRows rows or more on hipBLASLt (prefill_gemm_blas); repacked types on the wide-tile
// kernel that dequantizes in registers (launch_qf_gemm_wide) where the wide tile applies, else
// through an f16 copy in m->pf_wdeq; F16 and Q8_0 weights on launch_mfma. `defer` and *splits_out
// as launch_mfma's (split partials left in m->pf_part). *part_out: the library path's deferred
// partial (one, in m->pf_gu), else nullptr.
template <int EPI>
static int32_t prefill_gemm(aesir_model *m, hipStream_t s, const WMat &w, const void *A, int64_t M, int64_t K, int64_t N,
                            void *C, int64_t ldc, const char *name, bool defer = false, int64_t *splits_out = nullptr,
                            const float **part_out = nullptr) {
    if (M >= kBlasMinRows && m->pf_blas_ws) {
        const void *W = nullptr;
        if (w.type == AESIR_GGML_F16) {
            W = w.w;
        } else if (m->pf_wdeq && (qf_type(w.type) || (w.type == AESIR_GGML_Q8_0 && K % 32 == 0))) {
            // quantized: one f16 copy per chunk, with the rounding of the type's own GEMM kernels
            if (qf_type(w.type)) AESIR_TRY(launch_qf_dequant(s, wmat_qf(w), N, K, 1, nullptr, m->pf_wdeq, K));
            else AESIR_TRY(launch_q8_dequant_rows(s, w.w, w.s0, N, K, m->pf_wdeq));
            W = m->pf_wdeq;
        }
        if (W) {
            const int32_t rc = prefill_gemm_blas<EPI>(m, s, W, A, M, K, N, C, ldc, defer, splits_out, part_out);
            if (rc != AESIR_ERR_UNSUPPORTED) return rc;
        }
    }
    if (part_out) *part_out = nullptr;
    if (!qf_type(w.type))
        return launch_mfma<EPI>(s, A, M, K, w.w, N, C, ldc, m->pf_part, m->pf_part_floats, name, defer, splits_out,
                                w.type == AESIR_GGML_Q8_0 ? w.s0 : nullptr);
    // the 48-column tile is f16-only: plan as for Q8_0 weights (64 or 32 columns)
    if (const WidePlan wp = wide_plan(M, K, N, true); wp.nt) {
        int64_t splits = wp.splits;
        while (splits > 1 && splits * M * N > m->pf_part_floats) splits /= 2;
        AESIR_TRY(launch_qf_gemm_wide(s, EPI, wp.nt, A, M, K, wmat_qf(w), N, C, ldc, m->pf_part, splits));
        if (splits_out) *splits_out = splits;
        if (splits > 1 && !defer) {
            const int64_t blocks = (M * N + 255) / 256;
            hipLaunchKernelGGL(gemm_reduce_kernel<EPI>, dim3((unsigned)blocks), dim3(256), 0, s, (const float *)m->pf_part,
                               splits, M, N, (h16 *)C, ldc);
            AESIR_LAUNCH_CHECK("gemm_reduce_kernel");
        }
        return AESIR_OK;
    }
    AESIR_TRY(launch_qf_dequant(s, wmat_qf(w), N, K, 1, nullptr, m->pf_wdeq, K));
    return launch_mfma<EPI>(s, A, M, K, m->pf_wdeq, N, C, ldc, m->pf_part, m->pf_part_floats, name, defer, splits_out);
}

int64_t prefill_blas_min_rows() { return kBlasMinRows; }
int64_t prefill_blas_workspace() { return kBlasWorkspace; }

bool gemm_qf_wide_ok(int64_t M, int64_t K, int64_t N) { return wide_plan(M, K, N, true).nt != 0; }

int32_t launch_gemm_qf_mfma(aesir_ctx *ctx, const void *A, int64_t M, int64_t K, const QFMat &w, int64_t N, void *C) {
    const WidePlan wp = wide_plan(M, K, N, true);
    if (!wp.nt) return fail(AESIR_ERR_UNSUPPORTED, "gemm_qf_wide: shape not on the wide tile");
    int64_t splits = wp.splits;
    while (splits > 1 && splits * M * N > ctx->scratch.attn_part_floats) splits /= 2;
    AESIR_TRY(launch_qf_gemm_wide(ctx->stream, kEpiStore, wp.nt, A, M, K, w, N, C, N, ctx->scratch.attn_part, splits));
    if (splits > 1) {
        hipLaunchKernelGGL(gemm_reduce_kernel<kEpiStore>, dim3((unsigned)((M * N + 255) / 256)), dim3(256), 0,
                           ctx->stream, (const float *)ctx->scratch.attn_part, splits, M, N, (h16 *)C, N);
        AESIR_LAUNCH_CHECK("gemm_reduce_kernel");
    }
    return AESIR_OK;
}

int32_t launch_gemm_f16_mfma(aesir_ctx *ctx, const void *A, int64_t M, int64_t K, const void *B, int64_t N, void *C) {
    if (!mfma_shape_ok(A, M, K, B, N)) return launch_gemm_f16(ctx, A, M, K, B, N, C);
    return launch_mfma<kEpiStore>(ctx->stream, A, M, K, B, N, C, N, ctx->scratch.attn_part,
                                  ctx->scratch.attn_part_floats, "gemm_mfma_kernel");
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

// X[r] = token_embd[tokens[r]] (inference.mojo:452-467), one workgroup per row; the Q8_0 table
// variant writes f16(q * d) (the product is exact in f32, so one rounding, as f16(q) * d).
__global__ __launch_bounds__(kPThreads) void embed_rows_q8_kernel(const int8_t *__restrict__ q,
                                                                  const h16 *__restrict__ dsc, int64_t dim,
                                                                  const int64_t *__restrict__ tokens,
                                                                  h16 *__restrict__ X) {
    const int64_t t = tokens[blockIdx.x];
    const int8_t *src = q + t * dim;
    const h16 *ds = dsc + t * (dim / 32);
    h16 *dst = X + (int64_t)blockIdx.x * dim;
    for (int64_t c = threadIdx.x; c < dim; c += kPThreads) dst[c] = (h16)((float)src[c] * (float)ds[c / 32]);
}

// X[r] = token_embd[tokens[r]] (inference.mojo:452-467), one workgroup per row.
__global__ __launch_bounds__(kPThreads) void embed_rows_kernel(const h16 *__restrict__ table, int64_t dim,
                                                               const int64_t *__restrict__ tokens, h16 *__restrict__ X) {
    const h16 *src = table + tokens[blockIdx.x] * dim;
    h16 *dst = X + (int64_t)blockIdx.x * dim;
    for (int64_t c = threadIdx.x; c < dim; c += kPThreads) dst[c] = src[c];
}

int32_t launch_embed_rows(hipStream_t s, const WMat &e, int64_t dim, const int64_t *tokens, int64_t n, void *X) {
    if (n <= 0) return AESIR_OK;
    if (qf_type(e.type)) return launch_qf_dequant(s, wmat_qf(e), n, dim, 1, tokens, X, dim);
    if (e.type == AESIR_GGML_Q8_0)
        hipLaunchKernelGGL(embed_rows_q8_kernel, dim3((unsigned)n), dim3(kPThreads), 0, s, (const int8_t *)e.w,
                           (const h16 *)e.s0, dim, tokens, (h16 *)X);
    else
        hipLaunchKernelGGL(embed_rows_kernel, dim3((unsigned)n), dim3(kPThreads), 0, s, (const h16 *)e.w, dim, tokens,
                           (h16 *)X);
    AESIR_LAUNCH_CHECK("embed_rows_kernel");
    return AESIR_OK;
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

// Split-GEMM tails fused with the row kernel that follows them (one workgroup per row; the
// partials are summed in split order exactly as gemm_reduce_kernel does).
//   reduce_residual_norm_rows_kernel: X[m] = f16(f16(sum_z P[z][m]) + X[m]) (the residual
//     epilogue), then Xn[m] = rmsnorm(X[m]) with weight w (compute.mojo:2178-2204).
//   reduce_qkv_post_rows_kernel: QKV[m] = f16(sum_z P[z][m]) (the store epilogue) fed straight
//     into qkv_post_rows_kernel's RoPE and KV append.
constexpr int kRowVec = 8;  // columns per thread and pass (N % 8 == 0)
constexpr int kRowPasses = 2;  // rows up to 2 x 2048 columns keep their values in registers
// SPL > 0: the launch has exactly SPL splits, and every split's partials are requested before the
// first sum (one memory round trip instead of SPL); SPL = 0: any count, summed as loaded. Both
// add the splits in split order.
template <int SPL>
__global__ __launch_bounds__(kPThreads) void reduce_residual_norm_rows_kernel(const float *__restrict__ P,
                                                                              int64_t splits_rt, int64_t M, int64_t N,
                                                                              h16 *__restrict__ X, h16 *__restrict__ Xn,
                                                                              const h16 *__restrict__ w, float eps) {
    __shared__ float red[kPThreads / kWave];
    const int64_t splits = SPL > 0 ? SPL : splits_rt;
    const int64_t m = blockIdx.x;
    h16 *x = X + m * N;
    h16 *y = Xn + m * N;
    const bool keep = N <= (int64_t)kRowPasses * kPThreads * kRowVec;
    u32x4 xk0 = {0u, 0u, 0u, 0u}, xk1 = xk0;  // this thread's residual values of passes 0 and 1 (keep)
    float ss = 0.0f;
    int pass = 0;
    for (int64_t c0 = (int64_t)threadIdx.x * kRowVec; c0 < N; c0 += (int64_t)kPThreads * kRowVec, pass++) {
        const u32x4 xo = ld16(x + c0);
        float v[kRowVec];
#pragma unroll
        for (int e = 0; e < kRowVec; e++) v[e] = 0.0f;
        if (SPL > 0) {
            f32x4 a[SPL > 0 ? SPL : 1], b[SPL > 0 ? SPL : 1];
#pragma unroll
            for (int z = 0; z < SPL; z++) {
                const float *p = P + (z * M + m) * N + c0;
                a[z] = *reinterpret_cast<const f32x4 *>(p);
                b[z] = *reinterpret_cast<const f32x4 *>(p + 4);
            }
#pragma unroll
            for (int z = 0; z < SPL; z++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    v[e] += a[z][e];
                    v[4 + e] += b[z][e];
                }
        } else {
            for (int64_t z = 0; z < splits; z++) {
                const float *p = P + (z * M + m) * N + c0;
                const f32x4 a = *reinterpret_cast<const f32x4 *>(p), b = *reinterpret_cast<const f32x4 *>(p + 4);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    v[e] += a[e];
                    v[4 + e] += b[e];
                }
            }
        }
        u32x4 xn;
#pragma unroll
        for (int e = 0; e < kRowVec; e += 2) {
            const h16x2 old = as_h2(xo[e / 2]);
            const h16x2 nv = {hadd((h16)v[e], old.x), hadd((h16)v[e + 1], old.y)};
            xn[e / 2] = h2_bits(nv);
            const float f0 = (float)nv.x, f1 = (float)nv.y;
            ss = fmaf(f0, f0, ss);
            ss = fmaf(f1, f1, ss);
        }
        st16(x + c0, xn);
        if (pass == 0) xk0 = xn;
        else xk1 = xn;
    }
    ss = block_sum<kPThreads / kWave, false>(ss, red);
    const h16 inv = (h16)(1.0f / sqrtf(ss / (float)N + eps));
    pass = 0;
    for (int64_t c0 = (int64_t)threadIdx.x * kRowVec; c0 < N; c0 += (int64_t)kPThreads * kRowVec, pass++) {
        const u32x4 xv = !keep ? ld16(x + c0) : pass == 0 ? xk0 : xk1;
        const u32x4 wv = ld16(w + c0);
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const h16x2 a = as_h2(xv[e]), ww = as_h2(wv[e]);
            const h16x2 r = {hmul(hmul(a.x, inv), ww.x), hmul(hmul(a.y, inv), ww.y)};
            o[e] = h2_bits(r);
        }
        st16(y + c0, o);
    }
}

template <int SPL>
__global__ __launch_bounds__(kPThreads) void reduce_qkv_post_rows_kernel(
    const float *__restrict__ P, int64_t splits_rt, int64_t M, int64_t dim, int64_t kvd, int64_t hd, int64_t p0,
    int64_t max_seq, const h16x2 *__restrict__ rope, h16 *__restrict__ Q, h16 *__restrict__ kc, h16 *__restrict__ vc) {
    const int64_t splits = SPL > 0 ? SPL : splits_rt;
    const int64_t r = blockIdx.x, pos = p0 + r, slot = pos % max_seq;
    const int64_t N = dim + 2 * kvd, pairs = (dim + kvd) / 2;
    // grid.y workgroups share a row's pairs, so every thread sums one pair's partials
    for (int64_t j = (int64_t)blockIdx.y * kPThreads + threadIdx.x; j < N / 2; j += (int64_t)gridDim.y * kPThreads) {
        const int64_t col = 2 * j;
        float2 v = {0.0f, 0.0f};
        if (SPL > 0) {
            float2 t[SPL > 0 ? SPL : 1];
#pragma unroll
            for (int z = 0; z < SPL; z++) t[z] = *reinterpret_cast<const float2 *>(P + (z * M + r) * N + col);
#pragma unroll
            for (int z = 0; z < SPL; z++) {
                v.x += t[z].x;
                v.y += t[z].y;
            }
        } else {
            for (int64_t z = 0; z < splits; z++) {
                const float2 t = *reinterpret_cast<const float2 *>(P + (z * M + r) * N + col);
                v.x += t.x;
                v.y += t.y;
            }
        }
        const h16 a = (h16)v.x, b = (h16)v.y;
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
template <bool VEC>
__global__ __launch_bounds__(kWave) void prefill_attention_kernel(const h16 *__restrict__ Q, const h16 *__restrict__ kc,
                                                                  const h16 *__restrict__ vc, h16 *__restrict__ out,
                                                                  int64_t dim, int64_t kvd, int64_t hd, int64_t G,
                                                                  int64_t p0, int64_t max_seq, float scale) {
    __shared__ __align__(16) h16 qs[256];
    __shared__ float ps[kWave];
    const int lane = threadIdx.x;
    const int64_t r = blockIdx.x, h = blockIdx.y, g = h / G;
    const int64_t pos = p0 + r;
    const int64_t S = pos + 1 < max_seq ? pos + 1 : max_seq;
    const h16 *q = Q + r * dim + h * hd;
    for (int64_t d = lane; d < hd; d += kWave) qs[d] = q[d];
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
            if (VEC) {  // 16-byte K loads, v_dot2_f32_f16 against the q row in LDS
                for (int64_t i = 0; i < hd; i += 8) d = dot8(ld16(k + i), ld16(qs + i), d);
            } else {
                for (int64_t i = 0; i < hd; i++) d = fmaf((float)qs[i], (float)k[i], d);
            }
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

// The same attention for KV groups of 8 query heads (head_dim 64 or 128) or 4 (head_dim 128), one workgroup per
// (row, KV head): the G query heads that share a KV head are computed together, so each K/V row
// is loaded once per workgroup (whole 16-byte row segments) into LDS tiles of 128 positions
// instead of once per head and lane. Per tile: thread (head h, slot u) scores positions u,
// u + 256/G, ... (dot8 over the head dims in the same order as above), the G heads' f32 online
// softmax runs over their 256/G-thread groups, and thread (h, dim pair) accumulates P V from LDS.
constexpr int kAttTile = 128;
template <int HD, int G>
__global__ __launch_bounds__(kPThreads) void prefill_attention_tile_kernel(
    const h16 *__restrict__ Q, const h16 *__restrict__ kc, const h16 *__restrict__ vc, h16 *__restrict__ out,
    int64_t dim, int64_t kvd, int64_t p0, int64_t max_seq, float scale) {
    constexpr int TPH = kPThreads / G;        // threads per head (32 or 64)
    constexpr int NP = kAttTile / TPH;         // positions per thread per tile
    constexpr int NDP = HD / 2 / TPH;          // dim pairs per thread
    constexpr int KR = HD + 8;                 // padded K row (halves)
    constexpr int CH = HD / 8;                 // 16-byte chunks per row
    static_assert(NP >= 1 && NDP >= 1 && TPH <= kWave, "shape");
    __shared__ __align__(16) h16 ks[kAttTile][KR];
    __shared__ __align__(16) h16 vs[kAttTile][HD];
    __shared__ float ps[G][kAttTile];
    const int tid = threadIdx.x, h = tid / TPH, u = tid % TPH;
    const int64_t r = blockIdx.x, g = blockIdx.y;
    const int64_t pos = p0 + r;
    const int64_t S = pos + 1 < max_seq ? pos + 1 : max_seq;
    const int64_t head = g * G + h;
    u32x4 qr[CH];
    {
        const h16 *q = Q + r * dim + head * HD;
#pragma unroll
        for (int c = 0; c < CH; c++) qr[c] = ld16(q + 8 * c);
    }
    const h16 *Kg = kc + g * HD, *Vg = vc + g * HD;
    float m = -INFINITY, l = 0.0f, acc[NDP][2];
#pragma unroll
    for (int j = 0; j < NDP; j++) acc[j][0] = acc[j][1] = 0.0f;
    for (int64_t t0 = 0; t0 < S; t0 += kAttTile) {
        const int n = (int)(S - t0 < kAttTile ? S - t0 : kAttTile);
        __syncthreads();  // the previous tile's K, V and P are no longer read
        for (int e = tid; e < kAttTile * CH; e += kPThreads) {
            const int row = e / CH, c = e % CH;
            const int64_t p = t0 + (row < n ? row : 0);
            st16(&ks[row][8 * c], ld16(Kg + p * kvd + 8 * c));
            st16(&vs[row][8 * c], ld16(Vg + p * kvd + 8 * c));
        }
        __syncthreads();
        float sc[NP];
        float mt = -INFINITY;
#pragma unroll
        for (int j = 0; j < NP; j++) {
            const int row = u + j * TPH;
            float d = 0.0f;
#pragma unroll
            for (int c = 0; c < CH; c++) d = dot8(ld16(&ks[row][8 * c]), qr[c], d);
            sc[j] = row < n ? d * scale : -INFINITY;
            mt = fmaxf(mt, sc[j]);
        }
        mt = group_max<TPH>(mt);
        const float mn = fmaxf(m, mt);
        float lt = 0.0f;
#pragma unroll
        for (int j = 0; j < NP; j++) {
            const float pr = u + j * TPH < n ? expf(sc[j] - mn) : 0.0f;
            ps[h][u + j * TPH] = pr;
            lt += pr;
        }
        lt = group_sum<TPH>(lt);
        const float al = expf(m - mn);  // 0 on the first tile
        l = l * al + lt;
        m = mn;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NDP; j++) {
            const int dp = 2 * (u + j * TPH);
            float a0 = acc[j][0] * al, a1 = acc[j][1] * al;
            for (int t = 0; t < n; t++) {
                const float pr = ps[h][t];
                const h16x2 v = *reinterpret_cast<const h16x2 *>(&vs[t][dp]);
                a0 = fmaf(pr, (float)v.x, a0);
                a1 = fmaf(pr, (float)v.y, a1);
            }
            acc[j][0] = a0;
            acc[j][1] = a1;
        }
    }
    h16 *o = out + r * dim + head * HD;
#pragma unroll
    for (int j = 0; j < NDP; j++) {
        const int dp = 2 * (u + j * TPH);
        o[dp] = (h16)(acc[j][0] / l);
        o[dp + 1] = (h16)(acc[j][1] / l);
    }
}

// The same causal attention on the matrix cores, for chunks of many rows (no ring wrap inside the
// chunk). A 512-thread workgroup owns BQ = 128 / G consecutive rows and one KV head; wave w takes
// query head g G + w / (BQ / 16) on rows 16 (w % (BQ / 16)) .. + 15 of the block, so the 8 waves
// share every K/V tile of 64 keys, which the workgroup stages in LDS (the next tile's rows are
// requested into registers while the current one is used). Per tile and wave:
//   scores  S^T[64 keys][16 queries] = K Q^T on v_mfma_f32_16x16x32_f16 (A = K rows from LDS,
//           B = the wave's 16 query rows, held in registers): lane l holds query l % 16 and keys
//           16 t + 4 (l / 16) + i of sub-tile t; keys past a row's position are masked
//   softmax f32 online softmax per query: the lane's 16 values, then lanes l ^ 16, l ^ 32
//           (permlane swaps)
//   P V     O[16 queries][16 dims] += P V per 32-key step, A = the probabilities as they sit in
//           the score registers (slot 4 t + i of lane group q is key 16 t + 4 q + i), split into
//           two f16 terms (hi = f16(p), lo = f16(p - hi)) so that they keep f32 precision; B = V
//           read transposed from LDS with ds_read_b64_tr_b16 (V chunk c of row m at slot
//           c ^ 2 ((m / RPS) & SWM), which spreads the transposed reads over the banks)
// A tile entirely past a wave's last row is skipped by that wave. Scores and sums are f32, as in
// prefill_attention_tile_kernel; only the accumulation order differs.
typedef short short4_t __attribute__((ext_vector_type(4)));
constexpr int kPfBK = 64;            // keys per tile
constexpr int kPfWaves = 8;
constexpr int64_t kPfMfmaMinRows = 256;  // chunks from here on use the matrix-core attention
// Groups of 8 waves splitting a row block's key tiles (head_dim 64; at head_dim 128 the 1024-thread
// workgroup's 128-VGPR budget spills, so one group).
constexpr int kPfKeyGroups = 2;
template <int HD, int G, int KS>
__global__ __launch_bounds__(KS * kPfWaves * kWave) void prefill_attention_mfma_kernel(
    const h16 *__restrict__ Q, const h16 *__restrict__ kc, const h16 *__restrict__ vc, h16 *__restrict__ out,
    int64_t n, int64_t dim, int64_t kvd, int64_t p0, float scale) {
    constexpr int BQ = 16 * kPfWaves / G;  // rows per workgroup
    constexpr int RBLK = BQ / 16;          // 16-row blocks per head
    constexpr int NJ = HD / 32;            // score k-steps
    constexpr int NT = HD / 16;            // O dim tiles
    constexpr int KR = HD + 8;             // padded K row (halves)
    constexpr int RB = HD * 2;             // V row bytes
    constexpr int RPS = 256 / RB;          // V rows per 256 LDS bytes
    constexpr int SWM = RB / 32 - 1;
    constexpr int CH = HD / 8;             // 16-byte chunks per row
    constexpr int GT = kPfWaves * kWave;   // threads of a key group
    constexpr int NLD = kPfBK * CH / GT;   // K (and V) chunks per thread per tile
    constexpr int KB = kPfBK * KR * 2;     // K tile bytes (padded rows)
    constexpr int TB = KB + kPfBK * RB;    // K + V tile bytes of a key group
    static_assert(RBLK * G == kPfWaves && NLD >= 1 && NLD * GT == kPfBK * CH, "shape");
    static_assert(KS == 1 || kPfWaves * kWave * NT * 16 <= KS * TB, "the second group's O fits the tiles' LDS");
    __shared__ __align__(16) uint8_t smem[KS * TB];
    const int tid = threadIdx.x, lane = tid & 63;
    const int kg = tid / GT, gt = tid % GT, wave = gt >> 6;  // key group, thread and wave in it
    uint8_t *kbase = smem + kg * TB, *vs = kbase + KB;
    auto ks = [&](int row, int col) -> h16 * { return reinterpret_cast<h16 *>(kbase) + row * KR + col; };
    const int q4 = lane >> 4, c16 = lane & 15;
    const int64_t g = blockIdx.y;
    const int64_t rb0 = (int64_t)blockIdx.x * BQ;                 // first row of the workgroup
    const int64_t rlast = (rb0 + BQ < n ? rb0 + BQ : n) - 1;      // last valid row
    const int64_t kend = p0 + rlast + 1;                          // keys of the workgroup
    const int64_t ntile = (kend + kPfBK - 1) / kPfBK;
    const int64_t niter = (ntile + KS - 1) / KS;                  // tile rounds (group kg: tiles KS it + kg)
    const int hw = wave / RBLK;
    const int64_t r0w = rb0 + 16 * (wave % RBLK);                 // first row of the wave
    const int64_t rmax_w = r0w + 15 < rlast ? r0w + 15 : rlast;   // last valid row of the wave
    const int64_t head = g * G + hw;
    // this lane's query row (rows past the chunk are clamped: computed, never stored)
    const int64_t rq = r0w + c16 < rlast ? r0w + c16 : rlast;
    const int64_t kq = p0 + rq;  // last key the query sees
    u32x4 qb[NJ];
    {
        const h16 *qp = Q + rq * dim + head * HD + 8 * q4;
#pragma unroll
        for (int j = 0; j < NJ; j++) qb[j] = ld16(qp + 32 * j);
    }
    const h16 *Kg = kc + g * HD, *Vg = vc + g * HD;
    u32x4 kr[NLD], vr[NLD];
    auto load_tile = [&](int64_t t0) {  // rows past the workgroup's keys re-read its last key
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            const int e = gt + i * GT, row = e / CH, c = e % CH;
            const int64_t p = t0 + row < kend ? t0 + row : kend - 1;
            kr[i] = ld16(Kg + p * kvd + 8 * c);
            vr[i] = ld16(Vg + p * kvd + 8 * c);
        }
    };
    auto read_vt = [&](int nt, int m0) -> u32x2 {  // rows m0 + lane / 4, dims 16 nt + 4 (lane % 4) .. + 3
        const int m = m0 + (lane >> 2);
        const int c = 2 * nt + ((lane & 3) >> 1);
        const int sl = c ^ (2 * ((m / RPS) & SWM));
        return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                             (__attribute__((address_space(3))) short4_t *)(vs + m * RB + 16 * sl + 8 * (lane & 1))));
    };
    float m_run = -INFINITY, l_run = 0.0f;  // query c16 (the same in the four lane groups)
    f32x4 o[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) o[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    load_tile((int64_t)kg * kPfBK);
    for (int64_t it = 0; it < niter; it++) {
        const int64_t t0 = (it * KS + kg) * kPfBK;  // past kend: a surplus round of this group
        __syncthreads();  // the previous tiles are no longer read
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            const int e = gt + i * GT, row = e / CH, c = e % CH;
            st16(ks(row, 8 * c), kr[i]);
            st16(vs + row * RB + 16 * (c ^ (2 * ((row / RPS) & SWM))), vr[i]);
        }
        __syncthreads();
        if (it + 1 < niter) load_tile(t0 + KS * kPfBK);
        if (t0 > p0 + rmax_w) continue;  // every key of the tile is past this wave's rows
        f32x4 st[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            st[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < NJ; j++) st[t] = mfma16x16x32(ld16(ks(16 * t + c16, 32 * j + 8 * q4)), qb[j], st[t]);
        }
        float sv[4][4], mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t key = t0 + 16 * t + 4 * q4 + i;
                sv[t][i] = key <= kq ? st[t][i] * scale : -INFINITY;
                mx = fmaxf(mx, sv[t][i]);
            }
        mx = swap_pair_max<32>(swap_pair_max<16>(mx));
        // the tile holds a key the query sees (t0 <= p0 + rq for every row of the wave but
        // clamped rows past the chunk, which are never stored), so mx is finite
        const float mn = fmaxf(m_run, mx);
        const float al = expf(m_run - mn);   // 0 on the group's first tile
        float ps = 0.0f;
        u32x4 ph[2], pl[2];  // k-steps: keys of sub-tiles 2 kk and 2 kk + 1
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            h16 hi[8], lo[8];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float p = expf(sv[2 * kk + t][i] - mn);  // 0 where masked
                    ps += p;
                    hi[4 * t + i] = (h16)p;
                    lo[4 * t + i] = (h16)(p - (float)hi[4 * t + i]);
                }
            ph[kk] = u32x4{h2_bits(h16x2{hi[0], hi[1]}), h2_bits(h16x2{hi[2], hi[3]}), h2_bits(h16x2{hi[4], hi[5]}),
                           h2_bits(h16x2{hi[6], hi[7]})};
            pl[kk] = u32x4{h2_bits(h16x2{lo[0], lo[1]}), h2_bits(h16x2{lo[2], lo[3]}), h2_bits(h16x2{lo[4], lo[5]}),
                           h2_bits(h16x2{lo[6], lo[7]})};
        }
        ps = swap_pair_sum<16>(ps, ps);
        ps = swap_pair_sum<32>(ps, ps);
        l_run = l_run * al + ps;
        m_run = mn;
        // O rows of this lane are queries 4 q4 + i, whose factor sits in lane 4 q4 + i
        float alr[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            alr[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * (4 * q4 + i), __builtin_bit_cast(int, al)));
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
#pragma unroll
            for (int i = 0; i < 4; i++) o[nt][i] *= alr[i];
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
                const u32x2 v0 = read_vt(nt, 32 * kk), v1 = read_vt(nt, 32 * kk + 16);
                const u32x4 vb = u32x4{v0.x, v0.y, v1.x, v1.y};
                o[nt] = mfma16x16x32(ph[kk], vb, o[nt]);
                o[nt] = mfma16x16x32(pl[kk], vb, o[nt]);
            }
        }
    }
    if constexpr (KS == 2) {
        // group 1 hands (m, l, O) to the group-0 wave of the same rows and head through the tiles'
        // LDS: w = exp(m_g - max m) per query, l = sum w l_g, O = sum w O_g
        __syncthreads();  // every tile read is done
        f32x4 *ox = reinterpret_cast<f32x4 *>(smem);           // [wave][nt][lane]
        float *mx1 = reinterpret_cast<float *>(smem + kPfWaves * kWave * NT * 16);  // [wave][m: 16, l: 16]
        static_assert(kPfWaves * (kWave * NT * 16 + 32 * 4) <= KS * TB, "exchange fits");
        if (kg == 1) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) ox[(wave * NT + nt) * kWave + lane] = o[nt];
            if (q4 == 0) {
                mx1[wave * 32 + c16] = m_run;
                mx1[wave * 32 + 16 + c16] = l_run;
            }
        }
        __syncthreads();
        if (kg == 1) return;
        const float m1 = mx1[wave * 32 + c16], l1 = mx1[wave * 32 + 16 + c16];
        const float M = fmaxf(m_run, m1);   // m_run finite: group 0 holds tile 0
        const float e0 = expf(m_run - M), e1 = expf(m1 - M);  // e1 = 0 for a group without tiles
        l_run = l_run * e0 + l1 * e1;
        float e0r[4], e1r[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            e0r[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * (4 * q4 + i), __builtin_bit_cast(int, e0)));
            e1r[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * (4 * q4 + i), __builtin_bit_cast(int, e1)));
        }
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const f32x4 b = ox[(wave * NT + nt) * kWave + lane];
#pragma unroll
            for (int i = 0; i < 4; i++) o[nt][i] = o[nt][i] * e0r[i] + b[i] * e1r[i];
        }
    }
    float lr[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        lr[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * (4 * q4 + i), __builtin_bit_cast(int, l_run)));
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t r = r0w + 4 * q4 + i;
        if (r > rlast) continue;
        h16 *orow = out + r * dim + head * HD + c16;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) orow[16 * nt] = (h16)(o[nt][i] / lr[i]);
    }
}

// Launches prefill_attention_mfma_kernel for the shapes it is instantiated for;
// AESIR_ERR_UNSUPPORTED otherwise (the caller takes the tile kernels).
static int32_t launch_prefill_attention_mfma(hipStream_t s, int64_t hd, int64_t G, const h16 *Q, const h16 *kc,
                                             const h16 *vc, h16 *out, int64_t n, int64_t dim, int64_t kvd, int64_t p0,
                                             int64_t nkv, float scale) {
#define AESIR_PF_MMA(HDV, GV)                                                                                   \
    if (hd == HDV && G == GV) {                                                                                \
        constexpr int BQ = 16 * kPfWaves / GV, KS = HDV == 64 ? kPfKeyGroups : 1;                              \
        hipLaunchKernelGGL((prefill_attention_mfma_kernel<HDV, GV, KS>), dim3((unsigned)((n + BQ - 1) / BQ), (unsigned)nkv), \
                           dim3(KS * kPfWaves * kWave), 0, s, Q, kc, vc, out, n, dim, kvd, p0, scale);         \
        AESIR_LAUNCH_CHECK("prefill_attention_mfma_kernel");                                                   \
        return AESIR_OK;                                                                                       \
    }
    AESIR_PF_MMA(64, 8)
    AESIR_PF_MMA(64, 4)
    AESIR_PF_MMA(64, 2)
    AESIR_PF_MMA(64, 1)
    AESIR_PF_MMA(128, 8)
    AESIR_PF_MMA(128, 4)
    AESIR_PF_MMA(128, 2)
    AESIR_PF_MMA(128, 1)
#undef AESIR_PF_MMA
    return AESIR_ERR_UNSUPPORTED;
}

// act[i] = f16(up * silu(gate)) over interleaved [gate, up] pairs gu[2i], gu[2i + 1]
// (inference.mojo:257-260 on the gate/up GEMM rows as this build lays them out).
// VEC: n % 8 == 0 and 16-byte aligned buffers; each thread then takes 8 outputs (two 16-byte
// loads of pairs, one 16-byte store).
template <bool VEC>
__global__ __launch_bounds__(kPThreads) void swiglu_pairs_kernel(const h16 *__restrict__ gu, h16 *__restrict__ act,
                                                                 int64_t n) {
    if constexpr (VEC) {
        for (int64_t i = (int64_t)blockIdx.x * kPThreads + threadIdx.x; i < n / 8; i += (int64_t)gridDim.x * kPThreads) {
            const u32x4 a = ld16(gu + 16 * i), b = ld16(gu + 16 * i + 8);
            const unsigned w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            unsigned o[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const h16x2 p0 = as_h2(w[2 * j]), p1 = as_h2(w[2 * j + 1]);  // (gate, up) pairs
                o[j] = h2_bits(h16x2{hmul(p0.y, silu_h(p0.x)), hmul(p1.y, silu_h(p1.x))});
            }
            st16(act + 8 * i, u32x4{o[0], o[1], o[2], o[3]});
        }
    } else {
        for (int64_t i = (int64_t)blockIdx.x * kPThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kPThreads)
            act[i] = hmul(gu[2 * i + 1], silu_h(gu[2 * i]));
    }
}

static int32_t launch_swiglu_pairs(hipStream_t s, const void *gu, void *act, int64_t n) {
    const bool vec = n % 8 == 0 && ((uintptr_t)gu & 15) == 0 && ((uintptr_t)act & 15) == 0;
    int64_t g = ((vec ? n / 8 : n) + kPThreads - 1) / kPThreads;
    if (g > 65536) g = 65536;
    if (vec)
        hipLaunchKernelGGL(swiglu_pairs_kernel<true>, dim3((unsigned)g), dim3(kPThreads), 0, s, (const h16 *)gu,
                           (h16 *)act, n);
    else
        hipLaunchKernelGGL(swiglu_pairs_kernel<false>, dim3((unsigned)g), dim3(kPThreads), 0, s, (const h16 *)gu,
                           (h16 *)act, n);
    AESIR_LAUNCH_CHECK("swiglu_pairs_kernel");
    return AESIR_OK;
}

// ------------------------------------------------------------------ the batched pass

static const void *L0(const aesir_model *m) { return m->layers[0].qkv.w; }

// Every GEMM of a layer runs on the matrix cores when all four shapes qualify (arena buffers and
// weights are 256-byte aligned).
static bool prefill_mfma_ok(const aesir_model *m) {
    const int64_t d = m->cfg.dim, f = m->cfg.ffn, pr = m->pf_rows, qkv_n = d + 2 * m->kvd;
    const void *X = m->pf_xn;
    return mfma_shape_ok(X, pr, d, L0(m), qkv_n) && mfma_shape_ok(X, pr, d, L0(m), d) &&
           mfma_shape_ok(X, pr, d, L0(m), 2 * f) && mfma_shape_ok(X, pr, f, L0(m), d);
}

// Runs positions [p0, p0 + n) of tokens through every layer (n <= the model's prefill rows).
static int32_t prefill_chunk(aesir_model *m, const int64_t *tokens_host, int64_t p0, int64_t n) {
    const aesir_model_config &c = m->cfg;
    hipStream_t s = m->ctx->stream;
    const int64_t d = c.dim, kvd = m->kvd, f = c.ffn, hd = m->hd;
    const int64_t qkv_n = d + 2 * kvd;
    h16 *X = (h16 *)m->pf_x, *Xn = (h16 *)m->pf_xn, *QKV = (h16 *)m->pf_qkv, *Q = (h16 *)m->pf_q;
    h16 *ATT = (h16 *)m->pf_att, *ACT = (h16 *)m->pf_act;
    AESIR_HIP_TRY(hipMemcpyAsync(m->pf_tokens, tokens_host, (size_t)n * sizeof(int64_t), hipMemcpyHostToDevice, s));
    AESIR_TRY(launch_embed_rows(s, m->embd, d, (const int64_t *)m->pf_tokens, n, X));
    const bool mfma = prefill_mfma_ok(m);
    if (!mfma && !m->all_f16)
        return fail(AESIR_ERR_UNSUPPORTED, "prefill: quantized weights need the MFMA GEMM shapes (K %% 64 == 0)");
    const bool rowvec = d % kRowVec == 0;  // fused residual + norm rows need whole 8-column groups
    bool xn_ready = false;                 // Xn already holds this layer's attention-norm rows
    auto norm_rows = [&](const void *w) -> int32_t {
        hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3((unsigned)n), dim3(kPThreads), 0, s, X, Xn, d, (const h16 *)w,
                           c.rms_eps);
        AESIR_LAUNCH_CHECK("rmsnorm_rows_kernel");
        return AESIR_OK;
    };
    // residual GEMM into X, then X -> Xn normalized with `next_norm` (if any), fused when split
    auto residual_gemm = [&](const h16 *in, int64_t K, const WMat &w, const void *next_norm, const char *name) -> int32_t {
        int64_t splits = 1;
        const float *part = nullptr;
        AESIR_TRY(prefill_gemm<kEpiResidual>(m, s, w, in, n, K, d, X, d, name, next_norm && rowvec, &splits, &part));
        if (!next_norm) return AESIR_OK;
        if ((splits > 1 || part) && rowvec) {  // partials left for the fused residual + norm rows
            if (!part) part = m->pf_part;
#define AESIR_RRN(SV)                                                                                           \
    hipLaunchKernelGGL(reduce_residual_norm_rows_kernel<SV>, dim3((unsigned)n), dim3(kPThreads), 0, s,            \
                       part, splits, n, d, X, Xn, (const h16 *)next_norm, c.rms_eps)
            switch (splits) {
                case 1: AESIR_RRN(1); break;
                case 2: AESIR_RRN(2); break;
                case 3: AESIR_RRN(3); break;
                case 4: AESIR_RRN(4); break;
                case 5: AESIR_RRN(5); break;
                case 6: AESIR_RRN(6); break;
                case 7: AESIR_RRN(7); break;
                case 8: AESIR_RRN(8); break;
                default: AESIR_RRN(0); break;
            }
#undef AESIR_RRN
            AESIR_LAUNCH_CHECK("reduce_residual_norm_rows_kernel");
            return AESIR_OK;
        }
        return norm_rows(next_norm);
    };
    for (int64_t l = 0; l < c.n_layers; l++) {
        const ModelLayer &L = m->layers[l];
        h16 *kc = (h16 *)m->k_cache + l * c.ctx_len * kvd, *vc = (h16 *)m->v_cache + l * c.ctx_len * kvd;
        // attention block (inference.mojo:166-232)
        if (!xn_ready) AESIR_TRY(norm_rows(L.attn_norm));
        xn_ready = false;
        int64_t qkv_splits = 1;
        if (mfma && L.qkv_split > 0) {
            // a two-part Q/K/V: both parts dequantized into the f16 scratch matrix, then the F16 GEMM
            AESIR_TRY(launch_qf_dequant(s, wmat_qf(L.qkv), L.qkv_split, d, 1, nullptr, m->pf_wdeq, d));
            AESIR_TRY(launch_qf_dequant(s, wmat_qf(L.qkv_b), qkv_n - L.qkv_split, d, 1, nullptr,
                                        (h16 *)m->pf_wdeq + L.qkv_split * d, d));
            int32_t rc = AESIR_ERR_UNSUPPORTED;
            if (n >= kBlasMinRows && m->pf_blas_ws)
                rc = prefill_gemm_blas<kEpiStore>(m, s, m->pf_wdeq, Xn, n, d, qkv_n, QKV, qkv_n, false, &qkv_splits,
                                                  nullptr);
            if (rc == AESIR_ERR_UNSUPPORTED)
                AESIR_TRY(launch_mfma<kEpiStore>(s, Xn, n, d, m->pf_wdeq, qkv_n, QKV, qkv_n, m->pf_part,
                                                 m->pf_part_floats, "gemm_mfma_qkv", true, &qkv_splits));
            else if (rc != AESIR_OK)
                return rc;
        } else if (mfma) {
            AESIR_TRY(prefill_gemm<kEpiStore>(m, s, L.qkv, Xn, n, d, qkv_n, QKV, qkv_n, "gemm_mfma_qkv", true, &qkv_splits));
        } else {
            if (L.qkv_split > 0) return fail(AESIR_ERR_UNSUPPORTED, "prefill: two-part Q/K/V needs the matrix-core GEMM");
            AESIR_TRY(launch_gemm_f16(m->ctx, Xn, n, d, L.qkv.w, qkv_n, QKV));
        }
        if (qkv_splits > 1) {
            const dim3 qgrid((unsigned)n, (unsigned)((qkv_n / 2 + kPThreads - 1) / kPThreads));
#define AESIR_RQP(SV)                                                                                           \
    hipLaunchKernelGGL(reduce_qkv_post_rows_kernel<SV>, qgrid, dim3(kPThreads), 0, s, (const float *)m->pf_part, \
                       qkv_splits, n, d, kvd, hd, p0, c.ctx_len, (const h16x2 *)m->rope, Q, kc, vc)
            switch (qkv_splits) {
                case 2: AESIR_RQP(2); break;
                case 3: AESIR_RQP(3); break;
                case 4: AESIR_RQP(4); break;
                case 5: AESIR_RQP(5); break;
                case 6: AESIR_RQP(6); break;
                case 7: AESIR_RQP(7); break;
                case 8: AESIR_RQP(8); break;
                default: AESIR_RQP(0); break;
            }
#undef AESIR_RQP
            AESIR_LAUNCH_CHECK("reduce_qkv_post_rows_kernel");
        } else {
            hipLaunchKernelGGL(qkv_post_rows_kernel, dim3((unsigned)n), dim3(kPThreads), 0, s, QKV, d, kvd, hd, p0,
                               c.ctx_len, (const h16x2 *)m->rope, Q, kc, vc);
            AESIR_LAUNCH_CHECK("qkv_post_rows_kernel");
        }
        const int64_t G = c.n_heads / c.n_kv_heads;
        const dim3 tgrid((unsigned)n, (unsigned)c.n_kv_heads);
        bool att_done = false;
        if (n >= kPfMfmaMinRows && p0 + n <= c.ctx_len) {  // long chunk without ring wrap: matrix cores
            const int32_t rc = launch_prefill_attention_mfma(s, hd, G, Q, kc, vc, ATT, n, d, kvd, p0, c.n_kv_heads,
                                                             m->attn_scale);
            if (rc == AESIR_OK) att_done = true;
            else if (rc != AESIR_ERR_UNSUPPORTED) return rc;
        }
        if (!att_done) {
#define AESIR_PF_ATT(HDV, GV)                                                                                      \
    if (hd == HDV && G == GV)                                                                                     \
        hipLaunchKernelGGL((prefill_attention_tile_kernel<HDV, GV>), tgrid, dim3(kPThreads), 0, s, Q, kc, vc, ATT, d, \
                           kvd, p0, c.ctx_len, m->attn_scale);                                                   \
    else
            AESIR_PF_ATT(64, 8)
            AESIR_PF_ATT(128, 8)
            AESIR_PF_ATT(128, 4)
#undef AESIR_PF_ATT
            if (hd % 8 == 0)  // rows of K are then 16-byte aligned (kvd and the cache base are)
                hipLaunchKernelGGL(prefill_attention_kernel<true>, dim3((unsigned)n, (unsigned)c.n_heads), dim3(kWave), 0,
                                   s, Q, kc, vc, ATT, d, kvd, hd, c.n_heads / c.n_kv_heads, p0, c.ctx_len, m->attn_scale);
            else
                hipLaunchKernelGGL(prefill_attention_kernel<false>, dim3((unsigned)n, (unsigned)c.n_heads), dim3(kWave), 0,
                                   s, Q, kc, vc, ATT, d, kvd, hd, c.n_heads / c.n_kv_heads, p0, c.ctx_len, m->attn_scale);
            AESIR_LAUNCH_CHECK("prefill_attention_kernel");
        }
        // O projection + residual, then the feed-forward norm (inference.mojo:227-241)
        if (mfma) {
            AESIR_TRY(residual_gemm(ATT, d, L.o, L.ffn_norm, "gemm_mfma_o_residual"));
        } else {
            AESIR_TRY(launch_gemm_f16(m->ctx, ATT, n, d, L.o.w, d, Xn));
            AESIR_TRY(launch_residual_add(s, X, Xn, n * d));
            AESIR_TRY(norm_rows(L.ffn_norm));
        }
        // feed-forward block (inference.mojo:235-273); the down projection's tail also produces
        // the next layer's attention-norm rows
        if (mfma) {
            AESIR_TRY(prefill_gemm<kEpiSwiglu>(m, s, L.gu, Xn, n, d, 2 * f, ACT, f, "gemm_mfma_gate_up_swiglu"));
            const void *next_norm = l + 1 < c.n_layers ? m->layers[l + 1].attn_norm : nullptr;
            AESIR_TRY(residual_gemm(ACT, f, L.down, next_norm, "gemm_mfma_down_residual"));
            xn_ready = next_norm != nullptr;
        } else {
            // interleaved gate/up rows -> [n][2f] products, then the SwiGLU over the pairs
            if (!m->pf_gu) return fail(AESIR_ERR_UNSUPPORTED, "prefill: no gate/up buffer for the fallback GEMM");
            AESIR_TRY(launch_gemm_f16(m->ctx, Xn, n, d, L.gu.w, 2 * f, m->pf_gu));
            AESIR_TRY(launch_swiglu_pairs(s, m->pf_gu, ACT, n * f));
            AESIR_TRY(launch_gemm_f16(m->ctx, ACT, n, f, L.down.w, d, Xn));
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
    if (!m->all_f16 && !prefill_mfma_ok(m)) {
        // quantized weights in shapes the MFMA GEMM does not tile: the reference's prefill, one decode
        // step per position
        for (int64_t i = 0; i < n; i++) AESIR_TRY(model_step(m, tokens[i], start_pos + i, next));
        return AESIR_OK;
    }
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
