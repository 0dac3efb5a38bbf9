// Q8_0 GGUF-block matvec for gfx950 (gemm_q8_0, compute.mojo:1038-1065).
//
// Block layout: GGUF block_q8_0 = { f16 d; int8 qs[32] }, 34 bytes, packed, rows of K/32 blocks.
// One wave per output row. When K is a multiple of 64 each lane takes a pair of blocks (68
// bytes, 4-byte aligned) as 17 dword loads, so a wave reads one contiguous 4352-byte span;
// otherwise single blocks with 2-byte loads. Two activation types:
//   - f16 A (reference semantics): w = f16(f16(q) * d) per element, products summed in f32.
//   - f32 x (block matvec): y = sum over blocks of d * sum(q * x), all in f32.
#include "device.hpp"
#include "kernels.hpp"

namespace aesir {

constexpr int kQThreads = 256;
constexpr int kQRowsPerBlock = kQThreads / kWave;

template <bool F32X>
__device__ __forceinline__ float block_dot(const uint32_t *words, int byte0, const void *x, int64_t k0,
                                           float acc) {
    // words: the dwords covering this block; byte0: offset of the block inside them (0 or 2)
    auto byte_at = [&](int b) -> uint32_t { return (words[(byte0 + b) >> 2] >> (8 * ((byte0 + b) & 3))) & 0xffu; };
    const uint16_t dbits = (uint16_t)(byte_at(0) | (byte_at(1) << 8));
    const h16 d = bits_to_h(dbits);
    if (F32X) {
        const float *xf = reinterpret_cast<const float *>(x) + k0;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) s = fmaf((float)(int8_t)byte_at(2 + i), xf[i], s);
        return fmaf((float)d, s, acc);
    } else {
        const h16 *xh = reinterpret_cast<const h16 *>(x) + k0;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const h16 w = hmul((h16)(float)(int8_t)byte_at(2 + i), d);  // compute.mojo:1062-1063
            acc = fmaf((float)xh[i], (float)w, acc);
        }
        return acc;
    }
}

template <bool F32X, bool PAIRS>
__global__ __launch_bounds__(kQThreads) void q8_0_kernel(const uint8_t *__restrict__ blocks, int64_t N, int64_t K,
                                                         const void *__restrict__ xin, void *__restrict__ yout) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t n = (int64_t)blockIdx.x * kQRowsPerBlock + wave;
    const int64_t m = blockIdx.y;
    if (n >= N) return;
    const int64_t nb = K / 32;
    const uint8_t *row = blocks + n * nb * 34;
    const void *x = F32X ? (const void *)((const float *)xin + m * K) : (const void *)((const h16 *)xin + m * K);
    float acc = 0.0f;
    if (PAIRS) {
        const uint32_t *rw = reinterpret_cast<const uint32_t *>(row);
        for (int64_t p = lane; p < nb / 2; p += kWave) {
            uint32_t w[17];
#pragma unroll
            for (int i = 0; i < 17; i++) w[i] = rw[p * 17 + i];
            acc = block_dot<F32X>(w, 0, x, p * 64, acc);
            acc = block_dot<F32X>(w + 8, 2, x, p * 64 + 32, acc);
        }
    } else {
        for (int64_t b = lane; b < nb; b += kWave) {
            const uint16_t *bw = reinterpret_cast<const uint16_t *>(row + b * 34);
            uint32_t w[9];
#pragma unroll
            for (int i = 0; i < 8; i++) w[i] = (uint32_t)bw[2 * i] | ((uint32_t)bw[2 * i + 1] << 16);
            w[8] = bw[16];
            acc = block_dot<F32X>(w, 0, x, b * 32, acc);
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) {
        if (F32X)
            reinterpret_cast<float *>(yout)[m * N + n] = acc;
        else
            reinterpret_cast<h16 *>(yout)[m * N + n] = (h16)acc;
    }
}

template <bool F32X>
static int32_t q8_dispatch(hipStream_t s, const void *blocks, int64_t M, int64_t N, int64_t K, const void *x, void *y) {
    const dim3 grid((unsigned)((N + kQRowsPerBlock - 1) / kQRowsPerBlock), (unsigned)M);
    const bool pairs = (K % 64 == 0) && (((uintptr_t)blocks & 3) == 0);
    if (pairs)
        hipLaunchKernelGGL((q8_0_kernel<F32X, true>), grid, dim3(kQThreads), 0, s, (const uint8_t *)blocks, N, K, x, y);
    else
        hipLaunchKernelGGL((q8_0_kernel<F32X, false>), grid, dim3(kQThreads), 0, s, (const uint8_t *)blocks, N, K, x, y);
    AESIR_LAUNCH_CHECK("q8_0_kernel");
    return AESIR_OK;
}

int32_t launch_gemm_q8_0(hipStream_t s, const void *A, int64_t M, int64_t K, const void *blocks, int64_t N, void *C) {
    if (M > 65535) return fail(AESIR_ERR_UNSUPPORTED, "gemm_q8_0: more than 65535 rows of A");
    if (((uintptr_t)blocks & 1) != 0) return fail(AESIR_ERR_INVALID, "gemm_q8_0: blocks must be 2-byte aligned");
    return q8_dispatch<false>(s, blocks, M, N, K, A, C);
}

int32_t launch_q8_0_matvec_f32(hipStream_t s, const void *blocks, int64_t N, int64_t K, const float *x, float *y) {
    if (((uintptr_t)blocks & 1) != 0) return fail(AESIR_ERR_INVALID, "q8_0_matvec: blocks must be 2-byte aligned");
    return q8_dispatch<true>(s, blocks, 1, N, K, x, y);
}

}  // namespace aesir
