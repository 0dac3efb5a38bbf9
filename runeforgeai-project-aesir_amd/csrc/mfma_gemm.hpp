// Pieces shared by the batched-prefill GEMM kernels (f16 / Q8_0 weights in prefill.hip, repacked
// weights in quant.hip): the epilogues, the buffer-resource constant and the explicit wait count.
#pragma once

#include "device.hpp"

namespace aesir {

enum GemmEpi : int { kEpiStore = 0, kEpiResidual = 1, kEpiSwiglu = 2 };

// Third dword of a raw buffer resource (V#) on gfx9-family GPUs, gfx950 included.
constexpr int kBufferDword3 = 0x00020000;

// Applies the epilogue to output (m, n) with f32 value v; `partner` is the value of column n ^ 1
// in the same row (used by kEpiSwiglu: 2i gate, 2i + 1 up -> C[m][i] = f16(up * silu(gate))).
// kEpiStore: C[m][n] = f16(v); kEpiResidual: C[m][n] = f16(f16(v) + C[m][n]).
template <int EPI>
__device__ __forceinline__ void gemm_epilogue(h16 *C, int64_t ldc, int64_t M, int64_t N, int64_t m, int64_t n, float v,
                                              float partner) {
    if (EPI == kEpiSwiglu) {
        if ((n & 1) == 0 && m < M && n + 1 < N) C[m * ldc + n / 2] = hmul((h16)partner, silu_h((h16)v));
    } else if (m < M && n < N) {
        h16 *c = C + m * ldc + n;
        *c = EPI == kEpiResidual ? hadd((h16)v, *c) : (h16)v;
    }
}

// s_waitcnt immediate that waits until at most n vector-memory operations are outstanding
// (gfx9 encoding: vmcnt bits 3:0 and 15:14; expcnt and lgkmcnt left at their maxima).
constexpr int vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Rows of the activation chunk per wide-tile workgroup, the K chunk, and the LDS stages.
constexpr int kWideMT = 128, kWideKC = 128, kWideS = 3;
constexpr int kWideThreads = 8 * kWave;

}  // namespace aesir
