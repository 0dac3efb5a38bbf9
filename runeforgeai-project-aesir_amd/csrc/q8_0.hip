// Q8_0 GGUF-block matvec for gfx950 (gemm_q8_0, compute.mojo:1038-1065).
//
// Block layout: GGUF block_q8_0 = { f16 d; int8 qs[32] }, 34 bytes, packed, rows of K/32 blocks.
// One wave per output row. When K is a multiple of 64 each lane takes a pair of blocks (68
// bytes, 4-byte aligned) as 17 dword loads, so a wave reads one contiguous 4352-byte span;
// otherwise single blocks with 2-byte loads. Two activation types:
//   - f16 A (reference semantics): w = f16(f16(q) * d) per element, products summed in f32.
//   - f32 x (block matvec): y = sum over blocks of d * sum(q * x), all in f32.
#include <type_traits>

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

// Staged variant (rows of nb = K / 32 blocks with nb % 8 == 0, so every row span is a multiple of
// 16 bytes): the R rows of a workgroup are one contiguous byte range, copied into LDS with 16-byte
// buffer loads straight to LDS (a wave instruction moves 1 KB; every lane's request is coalesced;
// the pair kernel's 68-byte per-lane requests cost one address per 4 bytes). Thread t then owns
// block columns b = t, t + 256, ...: it loads x[32b, 32b + 32) once and applies it to block b of
// every row in LDS (9 dwords per block, 2-byte block offsets as above), so x is read once per
// workgroup. Per-row sums are reduced across the wave (recursive halving) and the 4 waves (LDS).
constexpr int kQSpanMax = 64 * 1024;  // LDS bytes of staged blocks per workgroup

constexpr int q8_vm_wait0() { return (7 << 4) | (15 << 8); }  // s_waitcnt vmcnt(0), others at max

// sum over the 32 elements of one block with its x (or A row) slice already in registers
template <bool F32X, class XT>
__device__ __forceinline__ float block_dot_regs(const uint32_t *words, int byte0, const XT (&xs)[32], float acc) {
    auto byte_at = [&](int b) -> uint32_t { return (words[(byte0 + b) >> 2] >> (8 * ((byte0 + b) & 3))) & 0xffu; };
    const h16 d = bits_to_h((uint16_t)(byte_at(0) | (byte_at(1) << 8)));
    if (F32X) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) s = fmaf((float)(int8_t)byte_at(2 + i), (float)xs[i], s);
        return fmaf((float)d, s, acc);
    } else {
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const h16 w = hmul((h16)(float)(int8_t)byte_at(2 + i), d);  // compute.mojo:1062-1063
            acc = fmaf((float)xs[i], (float)w, acc);
        }
        return acc;
    }
}

template <bool F32X, int R>
__global__ __launch_bounds__(kQThreads) void q8_0_staged_kernel(const uint8_t *__restrict__ blocks, int64_t N, int64_t K,
                                                                const void *__restrict__ xin, void *__restrict__ yout) {
    using XT = typename std::conditional<F32X, float, h16>::type;
    extern __shared__ __align__(16) uint8_t span[];
    __shared__ float red[kQRowsPerBlock * R];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t nb = K / 32, rowbytes = nb * 34;
    const int64_t n0 = (int64_t)blockIdx.x * R;
    const int64_t m = blockIdx.y;
    const int rows = (int)(N - n0 < R ? N - n0 : R);
    const int bytes = (int)(rows * rowbytes);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)(blocks + n0 * rowbytes), 0, bytes, 0x00020000);
    const int nchunks = bytes / 16;
    for (int c0 = wave * kWave; c0 < nchunks; c0 += kQThreads)  // chunks past the span read 0 (range check)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)(span + c0 * 16), 16,
                                                 (c0 + lane) * 16, 0, 0, 0);
    const XT *x = reinterpret_cast<const XT *>(xin) + m * K;
    const uint32_t *rw = reinterpret_cast<const uint32_t *>(span);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    XT xs[32];
    auto load_x = [&](int64_t b) {
        const int64_t bc = b < nb ? b : nb - 1;  // threads without a column load a valid one
#pragma unroll
        for (int i = 0; i < 32; i += 16 / (int)sizeof(XT))
            *reinterpret_cast<u32x4 *>(&xs[i]) = ld16(x + bc * 32 + i);
    };
    load_x(tid);  // with the copies in flight
    __builtin_amdgcn_s_waitcnt(q8_vm_wait0());
    __syncthreads();  // every wave's block copies are in LDS
    for (int64_t b = tid; b < nb; b += kQThreads) {
        if (b != tid) load_x(b);
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (r < rows) {
                const int off = (int)(r * rowbytes + b * 34);
                uint32_t w[9];
#pragma unroll
                for (int i = 0; i < 9; i++) w[i] = rw[(off >> 2) + i];
                // realign to the block's first byte (offset 0 or 2 in the first dword) with
                // v_alignbyte, so that byte indices stay compile-time constants
                const unsigned sh = (unsigned)(off & 3);
#pragma unroll
                for (int i = 0; i < 8; i++) w[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
                w[8] = w[8] >> (8 * sh);
                acc[r] = block_dot_regs<F32X>(w, 0, xs, acc[r]);
            }
        }
    }
    wave_multi_sum<R>(acc, lane);
    constexpr int GW = kWave / R;
    if ((lane & (GW - 1)) == 0) red[wave * R + lane / GW] = acc[0];
    __syncthreads();
    if (tid < rows) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kQRowsPerBlock; w++) v += red[w * R + tid];
        if (F32X)
            reinterpret_cast<float *>(yout)[m * N + n0 + tid] = v;
        else
            reinterpret_cast<h16 *>(yout)[m * N + n0 + tid] = (h16)v;
    }
}

template <bool F32X>
static int32_t q8_dispatch(hipStream_t s, const void *blocks, int64_t M, int64_t N, int64_t K, const void *x, void *y) {
    const int64_t nb = K / 32, rowbytes = nb * 34;
    if (K % 32 == 0 && nb % 8 == 0 && ((uintptr_t)blocks & 15) == 0 && ((uintptr_t)x & 15) == 0 && rowbytes <= kQSpanMax &&
        N * rowbytes < ((int64_t)1 << 31)) {
        const int r = 8 * rowbytes <= kQSpanMax ? 8 : 4 * rowbytes <= kQSpanMax ? 4 : 2 * rowbytes <= kQSpanMax ? 2 : 1;
        const unsigned lds = (unsigned)((r * rowbytes + 1023) / 1024 * 1024);  // whole 1 KB copy instructions
        const dim3 grid((unsigned)((N + r - 1) / r), (unsigned)M);
#define AESIR_Q8_STAGED(RV)                                                                                    \
        if (r == RV) {                                                                                         \
            if (lds > 65536)                                                                                   \
                AESIR_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(q8_0_staged_kernel<F32X, RV>),  \
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));      \
            hipLaunchKernelGGL((q8_0_staged_kernel<F32X, RV>), grid, dim3(kQThreads), lds, s,                   \
                               (const uint8_t *)blocks, N, K, x, y);                                           \
        }
        AESIR_Q8_STAGED(8)
        AESIR_Q8_STAGED(4)
        AESIR_Q8_STAGED(2)
        AESIR_Q8_STAGED(1)
#undef AESIR_Q8_STAGED
        AESIR_LAUNCH_CHECK("q8_0_staged_kernel");
        return AESIR_OK;
    }
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
