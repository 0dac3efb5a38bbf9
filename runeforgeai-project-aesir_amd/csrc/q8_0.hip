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

// f32 matvec on rows of nb = 64, 128, 256, 448 or 512 blocks: x as integer digits, persistent
// workgroups with an LDS ring.
//   - Thread t owns block column b = t % nb of a row phase ph = t / nb (PH = 64 NW / nb phases).
//     It holds its 32 x values as a fixed-point integer v = rint(x * 2^(29 - e)), e = ilogb of the
//     block's largest |x| (|v| <= 2^30, rounding error <= 2^(e - 30) <= 2^-30 of that largest
//     |x|), split into four signed 8-bit digits v = d0 + 2^8 d1 + 2^16 d2 + 2^24 d3 packed four to
//     a dword (32 registers).
//   - Per row the block's 32 quants meet each digit in 8 v_dot4_i32_i8 (exact integer sums, each
//     below 2^20 in magnitude); the four sums are recombined exactly in f64 (below 2^44), then
//     multiplied by the block scale d and by 2^(e - 29) and rounded to f32. So a block's value is
//     within 2^-30 * max|x_blk| * sum|d q| (plus one f32 rounding) of the exact block dot product;
//     the block values are summed in f32. A block whose x holds an inf or NaN takes the plain f32
//     product instead, so such inputs propagate as in the f32 formula.
//   - Workgroup g handles row groups g, g + G, ... of R = PH RT rows; each group's contiguous byte
//     span is copied by 16-byte buffer loads with the LDS destination into one of S stages, S - 1
//     groups ahead of the one being summed (every wave issues P one-kilobyte copies per group, the
//     range check zero-fills past the matrix, so the vmcnt waits are exact counts).
constexpr int kCus = 256;  // MI355X compute units (the persistent grid's size unit)
constexpr int kQDirectRpw = 64;  // rows per workgroup of q8_0_direct_kernel (its LDS row sums)
// 16 bytes loaded from a 4-byte aligned address (gfx950 serves unaligned vector loads)
typedef unsigned int u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
constexpr int q8_vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// The four signed 8-bit digit planes of a block's 32 x values (see above): v = rint(x 2^(29 - e)),
// u = v + 0x808080 has the bytes d0 + 128, d1 + 128, d2 + 128 (each d_j in [-128, 127], d_j = v's
// nearest-digit recurrence) and the signed top digit d3 = floor(u / 2^24), |d3| <= 64; a 4 x 4 byte
// transpose (v_perm_b32) gathers digit j of four x values into dg[j][w], and the xor with 0x80 per
// byte turns d_j + 128 back into d_j. plain: the block holds an inf or NaN (then dg is zero).
__device__ __forceinline__ void x_digits(const float *xb, int (&dg)[4][8], int &ex, bool &plain) {
    float xv[32];
#pragma unroll
    for (int i = 0; i < 32; i += 4) *reinterpret_cast<u32x4 *>(&xv[i]) = ld16(xb + i);
    float m = 0.0f;
    plain = false;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        m = fmaxf(m, fabsf(xv[i]));
        plain |= !(fabsf(xv[i]) <= 3.402823466e38f);  // inf or NaN
    }
    ex = m > 0.0f && !plain ? ilogbf(m) : 0;
#pragma unroll
    for (int w = 0; w < 8; w++) {
        unsigned u[4];
#pragma unroll
        for (int k = 0; k < 4; k++)
            u[k] = plain ? 0x808080u : (unsigned)((int)rintf(ldexpf(xv[4 * w + k], 29 - ex)) + 0x808080);  // |v| <= 2^30
        const unsigned t01l = __builtin_amdgcn_perm(u[1], u[0], 0x05010400u), t01h = __builtin_amdgcn_perm(u[1], u[0], 0x07030602u);
        const unsigned t23l = __builtin_amdgcn_perm(u[3], u[2], 0x05010400u), t23h = __builtin_amdgcn_perm(u[3], u[2], 0x07030602u);
        dg[0][w] = (int)(__builtin_amdgcn_perm(t23l, t01l, 0x05040100u) ^ 0x80808080u);
        dg[1][w] = (int)(__builtin_amdgcn_perm(t23l, t01l, 0x07060302u) ^ 0x80808080u);
        dg[2][w] = (int)(__builtin_amdgcn_perm(t23h, t01h, 0x05040100u) ^ 0x80808080u);
        dg[3][w] = (int)__builtin_amdgcn_perm(t23h, t01h, 0x07060302u);
    }
}

template <int NW, int PH, int RT, int S, int P>
__global__ __launch_bounds__(NW * 64) void q8_0_digits_kernel(const uint8_t *__restrict__ blocks, int64_t N,
                                                              int64_t rowbytes, const float *__restrict__ x,
                                                              float *__restrict__ y) {
    extern __shared__ __align__(16) uint8_t ring[];
    constexpr int T = NW * 64, NB = T / PH, R = PH * RT, WPP = NW / PH;
    constexpr int kStage = P * NW * 1024, kYs = 16;
    __shared__ float red[NW * RT];
    __shared__ float ys[kYs * R];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int b = tid % NB, ph = tid / NB;
    const int64_t ng = (N + R - 1) / R;
    const float *xb = x + 32 * b;
    int dg[4][8];
    int ex;
    bool plain;
    {
        float xv[32];
#pragma unroll
        for (int i = 0; i < 32; i += 4) *reinterpret_cast<u32x4 *>(&xv[i]) = ld16(xb + i);
        float m = 0.0f;
        plain = false;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            m = fmaxf(m, fabsf(xv[i]));
            plain |= !(fabsf(xv[i]) <= 3.402823466e38f);  // inf or NaN
        }
        ex = m > 0.0f && !plain ? ilogbf(m) : 0;
#pragma unroll
        for (int w = 0; w < 8; w++) {
            unsigned p[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int v = plain ? 0 : (int)rintf(ldexpf(xv[4 * w + k], 29 - ex));  // |v| <= 2^30
                const int d0 = (int)(int8_t)(v & 0xff);
                const int r1 = (v - d0) >> 8;
                const int d1 = (int)(int8_t)(r1 & 0xff);
                const int r2 = (r1 - d1) >> 8;
                const int d2 = (int)(int8_t)(r2 & 0xff);
                const int d3 = (r2 - d2) >> 8;  // |d3| <= 64
                p[0] |= (unsigned)(d0 & 0xff) << (8 * k);
                p[1] |= (unsigned)(d1 & 0xff) << (8 * k);
                p[2] |= (unsigned)(d2 & 0xff) << (8 * k);
                p[3] |= (unsigned)(d3 & 0xff) << (8 * k);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) dg[j][w] = (int)p[j];
        }
    }
    // the digits are in registers before the first copy is issued (no x load left in flight)
#pragma unroll
    for (int w = 0; w < 8; w++) asm volatile("" : "+v"(dg[0][w]), "+v"(dg[1][w]), "+v"(dg[2][w]), "+v"(dg[3][w]));
    auto issue = [&](int64_t g, int stage) {
        int64_t rows = N - g * R;
        rows = rows < 0 ? 0 : rows > R ? R : rows;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(blocks + (rows > 0 ? g * R * rowbytes : 0)), 0, (int)(rows * rowbytes), 0x00020000);
#pragma unroll
        for (int j = 0; j < P; j++) {
            const int c0 = (j * NW + wave) * kWave;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (__attribute__((address_space(3))) void *)(ring + stage * kStage + c0 * 16), 16, (c0 + lane) * 16, 0,
                0, 0);
        }
    };
    const int64_t g0 = blockIdx.x, gs = gridDim.x;
#pragma unroll
    for (int s = 0; s < S - 1; s++) issue(g0 + s * gs, s);
    const int bo = 34 * b, sh = bo & 3;
    // Row results wait in LDS and go out kYs groups at a time: a global store in the loop would
    // make the next group's vmcnt wait include its write acknowledgement.
    auto flush = [&](int cnt, int64_t g_end) {
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        for (int i = tid; i < cnt * R; i += T) {
            const int64_t n = (g_end - (int64_t)(cnt - 1 - i / R) * gs) * R + i % R;
            if (n < N) y[n] = ys[i];
        }
    };
    int stage = 0, it = 0;
    int64_t last = g0;
    for (int64_t g = g0; g < ng; g += gs) {
        issue(g + (S - 1) * gs, stage == 0 ? S - 1 : stage - 1);  // the stage summed one group ago
        __builtin_amdgcn_s_waitcnt(q8_vm_wait((S - 1) * P));       // this wave's copies of group g ...
        __builtin_amdgcn_s_barrier();                              // ... and every other wave's
        const uint32_t *st = reinterpret_cast<const uint32_t *>(ring + stage * kStage);
        float acc[RT];
        auto block_words = [&](int rr, uint32_t (&w)[9]) {  // block b of row ph + PH rr, from its first byte
            const int wi = ((ph + PH * rr) * (int)rowbytes + bo) >> 2;
#pragma unroll
            for (int i = 0; i < 9; i++) w[i] = st[wi + i];
#pragma unroll
            for (int i = 0; i < 8; i++) w[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
            w[8] = w[8] >> (8 * sh);
        };
        if (!plain) {
#pragma unroll
            for (int rr = 0; rr < RT; rr++) {
                uint32_t w[9];
                block_words(rr, w);
                int s0 = 0, s1 = 0, s2 = 0, s3 = 0;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int q = (int)__builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);  // quants 4i .. 4i + 3
                    s0 = __builtin_amdgcn_sdot4(q, dg[0][i], s0, false);
                    s1 = __builtin_amdgcn_sdot4(q, dg[1][i], s1, false);
                    s2 = __builtin_amdgcn_sdot4(q, dg[2][i], s2, false);
                    s3 = __builtin_amdgcn_sdot4(q, dg[3][i], s3, false);
                }
                // exact in f64: |s_j| < 2^20, the sum < 2^44
                const double v = fma((double)s3, 16777216.0, fma((double)s2, 65536.0, fma((double)s1, 256.0, (double)s0)));
                acc[rr] = (float)ldexp(v * (double)bits_to_h((uint16_t)(w[0] & 0xffff)), ex - 29);
            }
        } else {
#pragma unroll
            for (int rr = 0; rr < RT; rr++) {
                uint32_t w[9];
                block_words(rr, w);
                float v = 0.0f;
#pragma unroll
                for (int i = 0; i < 32; i++) {
                    const int bb = 2 + i;
                    v = fmaf((float)(int8_t)((w[bb >> 2] >> (8 * (bb & 3))) & 0xff), xb[i], v);
                }
                acc[rr] = (float)bits_to_h((uint16_t)(w[0] & 0xffff)) * v;
            }
        }
        wave_multi_sum<RT>(acc, lane);
        constexpr int GW = kWave / RT;
        if ((lane & (GW - 1)) == 0) red[wave * RT + lane / GW] = acc[0];
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the row sums are in LDS
        __builtin_amdgcn_s_barrier();
        if (tid < R) {  // row g R + tid: phase tid % PH, waves of that phase
            const int p = tid % PH, ri = tid / PH;
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < WPP; w++) v += red[(p * WPP + w) * RT + ri];
            ys[(it % kYs) * R + tid] = v;
        }
        stage = stage + 1 == S ? 0 : stage + 1;
        if (++it % kYs == 0) flush(kYs, g);
        last = g;
    }
    __builtin_amdgcn_s_waitcnt(q8_vm_wait(0));  // no copy may land in LDS after the workgroup ends
    if (it % kYs) flush(it % kYs, last);
}

// The same integer-digit arithmetic with the weights loaded straight into registers (no LDS
// staging), for rows of nb = 64 WPR blocks.
//   - Lane l of wave w owns block column b = 64 (w % WPR) + l, so a wave covers 64 consecutive
//     blocks (2176 contiguous bytes) of a row and WPR waves cover the row; the workgroup's PH row
//     phases (w / WPR) take its rows.
//   - Per row a lane loads 16 + 16 + 4 bytes: the 32 bytes from the 4-byte aligned word at or below
//     its block's quants (34 b + 2: two bytes into a word for an even b, on a word boundary for an
//     odd one) and one more word (the last two quants of an even b, the scale d of an odd b). The
//     lanes of one instruction read 64 blocks' bytes 34 apart: every cache line of the wave's span
//     is requested by each instruction that touches it, which the L1 absorbs; HBM sees the row once.
//   - Rows are dealt out across the grid: at step k workgroup g's phase p takes row
//     (k G + g) PH + p (G workgroups), so the grid sweeps the matrix front to back together
//     instead of running G separate streams.
//   - D rows are in flight per wave: row step k + D is requested as soon as step k has been
//     consumed, into the registers step k used (the loop is unrolled D times, so the wait before a
//     row counts exactly the loads issued after it). The first D rows are requested before x is
//     read and turned into digits.
//   - A row's 64 block values per wave are summed by recursive halving (two rows at a time); the
//     wave sums go to LDS and, after the workgroup's last row, WPR of them make each row's y. No
//     barrier runs before the end.
template <int WPR, int PH, int D>
__global__ __launch_bounds__(WPR * PH * 64) void q8_0_direct_kernel(const uint8_t *__restrict__ blocks, int64_t N,
                                                                   int64_t rowbytes, int64_t rpw,
                                                                   const float *__restrict__ x, float *__restrict__ y) {
    constexpr int NW = WPR * PH;
    static_assert(D % 2 == 0 && D >= 2 && D <= 8, "rows in flight: an even count, 3 loads each under vmcnt's 63");
    __shared__ float part[kQDirectRpw][WPR];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = wave % WPR, ph = wave / WPR;
    const int b = 64 * c + lane;
    // row of step k of phase p: (k G + g) PH + p, so that at step k the whole grid reads rows
    // [k G PH, (k + 1) G PH): one sweep through the matrix instead of G separate streams
    const int64_t G = gridDim.x, g = blockIdx.x;
    auto row_of = [&](int64_t k, int p) { return (k * G + g) * PH + p; };
    const int nmine = row_of(0, ph) < N ? (int)((N - 1 - row_of(0, ph)) / (G * PH)) + 1 : 0;  // rows of this wave

    const float *xb = x + 32 * b;
    int dg[4][8];  // x digits, ex and plain: set after the first weight requests (x_digits below)
    int ex = 0;
    bool plain = false;
    // Quants of block b start at byte 34 b + 2: at byte 2 of the 4-byte aligned word at 34 b for
    // an even b, at a word boundary for an odd one. A lane loads the 32 bytes from the aligned word
    // at or below its quants (A, B) and one word C: the one after them for an even b (its last two
    // quants), the one holding d for an odd b (d sits just before its quants).
    const bool odd = b & 1;
    const int qoff = odd ? 34 * b + 2 : 34 * b, coff = odd ? 34 * b - 2 : 34 * b + 32;
    const unsigned qs = odd ? 0u : 2u;  // byte shift from the loaded words to the quants
    struct Row {
        u32x4 a, bq;
        uint32_t c;
    };
    auto load = [&](int k, Row &rw) {  // row k of this wave (rows past the matrix re-read the last one)
        int64_t r = row_of(k, ph);
        r = r < N ? r : N - 1;
        const uint8_t *p = blocks + r * rowbytes;
        rw.a = *reinterpret_cast<const u32x4_a4 *>(p + qoff);
        rw.bq = *reinterpret_cast<const u32x4_a4 *>(p + qoff + 16);
        rw.c = *reinterpret_cast<const uint32_t *>(p + coff);
    };
    auto value = [&](const Row &rw) -> float {  // block b of the row
        const uint32_t w[9] = {rw.a.x, rw.a.y, rw.a.z, rw.a.w, rw.bq.x, rw.bq.y, rw.bq.z, rw.bq.w, rw.c};
        const h16 d = bits_to_h((uint16_t)(odd ? rw.c >> 16 : rw.a.x & 0xffff));
        uint32_t q[8];  // quants 4i .. 4i + 3 (for an odd b, alignbyte by 0 ignores its high word)
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], qs);
        if (!plain) {
            int s0 = 0, s1 = 0, s2 = 0, s3 = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                s0 = __builtin_amdgcn_sdot4((int)q[i], dg[0][i], s0, false);
                s1 = __builtin_amdgcn_sdot4((int)q[i], dg[1][i], s1, false);
                s2 = __builtin_amdgcn_sdot4((int)q[i], dg[2][i], s2, false);
                s3 = __builtin_amdgcn_sdot4((int)q[i], dg[3][i], s3, false);
            }
            // exact in f64: |s_j| < 2^20, the sum < 2^44
            const double v = fma((double)s3, 16777216.0, fma((double)s2, 65536.0, fma((double)s1, 256.0, (double)s0)));
            return (float)ldexp(v * (double)d, ex - 29);
        }
        float v = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) v = fmaf((float)(int8_t)((q[i >> 2] >> (8 * (i & 3))) & 0xff), xb[i], v);
        return (float)d * v;
    };
    // two rows' block values -> their wave sums (lanes 0 .. 31 hold row 0's, 32 .. 63 row 1's)
    auto emit = [&](int k, float v0, float v1) {
        float acc[2] = {v0, v1};
        wave_multi_sum<2>(acc, lane);
        if ((lane & 31) == 0) {
            const int kk = k + (lane >> 5);
            if (kk < nmine) part[kk * PH + ph][c] = acc[0];
        }
    };
    // The first D rows are requested before x, so the weight stream starts at once; x and the
    // digits follow (waiting for x waits for those rows too, which the first row needs anyway).
    Row rr[D];
#pragma unroll
    for (int j = 0; j < D; j++) {
        load(j, rr[j]);
        __builtin_amdgcn_sched_barrier(0);
    }
    x_digits(xb, dg, ex, plain);
    __builtin_amdgcn_sched_barrier(0);
    for (int k = 0; k < nmine; k += D) {
#pragma unroll
        for (int j = 0; j < D; j += 2) {
            const float v0 = value(rr[j]);
            __builtin_amdgcn_sched_barrier(0);
            load(k + D + j, rr[j]);
            __builtin_amdgcn_sched_barrier(0);
            const float v1 = value(rr[j + 1]);
            __builtin_amdgcn_sched_barrier(0);
            load(k + D + j + 1, rr[j + 1]);
            __builtin_amdgcn_sched_barrier(0);
            emit(k + j, v0, v1);
        }
    }
    __builtin_amdgcn_s_waitcnt(q8_vm_wait(0));  // the loads past the last row, before the barrier
    __syncthreads();
    for (int i = tid; i < rpw; i += NW * 64) {
        const int64_t r = row_of(i / PH, i % PH);
        if (r >= N) continue;
        float v = 0.0f;
#pragma unroll
        for (int j = 0; j < WPR; j++) v += part[i][j];
        y[r] = v;
    }
}

template <int WPR, int PH, int D>
static int32_t launch_direct(hipStream_t s, const void *blocks, int64_t N, int64_t rowbytes, const float *x, float *y,
                             int wg_per_cu) {
    // rpw: rows per workgroup, a multiple of PH (row steps x phases)
    int64_t steps = (N + (int64_t)kCus * wg_per_cu * PH - 1) / ((int64_t)kCus * wg_per_cu * PH);
    if (steps * PH > kQDirectRpw) steps = kQDirectRpw / PH;
    const int64_t rpw = steps * PH;
    const int64_t grid = (N + rpw - 1) / rpw;
    hipLaunchKernelGGL((q8_0_direct_kernel<WPR, PH, D>), dim3((unsigned)grid), dim3(WPR * PH * 64), 0, s,
                       (const uint8_t *)blocks, N, rowbytes, rpw, x, y);
    AESIR_LAUNCH_CHECK("q8_0_direct_kernel");
    return AESIR_OK;
}

template <int NW, int PH, int RT, int S, int P>
static int32_t launch_digits(hipStream_t s, const void *blocks, int64_t N, int64_t rowbytes, const float *x, float *y,
                             int wg_per_cu) {
    constexpr int R = PH * RT;
    static_assert(P * NW * 1024 >= 0, "stage size");
    if ((int64_t)R * rowbytes + 16 > (int64_t)P * NW * 1024) return fail(AESIR_ERR_INVALID, "q8_0_matvec: stage too small");
    const unsigned lds = (unsigned)(S * P * NW * 1024);
    const void *fn = reinterpret_cast<const void *>(q8_0_digits_kernel<NW, PH, RT, S, P>);
    static std::atomic<uint64_t> lds_set{0};
    if (lds > 65536) AESIR_TRY(raise_lds_limit(fn, (int)lds, lds_set));
    const int64_t ng = (N + R - 1) / R;
    const int64_t grid = ng < (int64_t)kCus * wg_per_cu ? ng : (int64_t)kCus * wg_per_cu;
    hipLaunchKernelGGL((q8_0_digits_kernel<NW, PH, RT, S, P>), dim3((unsigned)grid), dim3(NW * 64), lds, s,
                       (const uint8_t *)blocks, N, rowbytes, x, y);
    AESIR_LAUNCH_CHECK("q8_0_digits_kernel");
    return AESIR_OK;
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
    const int64_t nb = K / 32, rowbytes = nb * 34;
    // Digit kernel shapes (rows of 64 .. 512 blocks, one thread per block column). Stage sizes and
    // workgroups per CU measured on MI355X at 14336 x 4096 (2 per CU, 2 stages: 13.8 us against 17.5
    // for the staged kernel) and 4096 x 14336 (1 per CU, 3 stages: 14.8 us against 19.6).
    if (K % 32 == 0 && ((uintptr_t)blocks & 15) == 0 && ((uintptr_t)x & 15) == 0 && N * rowbytes < ((int64_t)1 << 31)) {
        // Llama's 4096- and 14336-long rows: the register-direct kernel, one workgroup per CU
        // (measured on MI355X, 32 calls graph-replayed, weights past the MALL: 14336 x 4096 12.6 us
        // against 15.2 for the LDS-ring kernel, 4096 x 14336 14.2 against 16.9; 2 or 4 workgroups
        // per CU, 2 row phases for the 14336-long rows, or 2 rows in flight for the 4096-long rows
        // measured 13 to 22 us)
        switch (nb) {
            case 64: return launch_digits<4, 4, 2, 2, 5>(s, blocks, N, rowbytes, x, y, 2);     // 8 rows, 17 KB
            case 128: return launch_direct<2, 2, 4>(s, blocks, N, rowbytes, x, y, 1);
            case 256: return launch_digits<4, 1, 4, 2, 9>(s, blocks, N, rowbytes, x, y, 2);    // 4 rows, 34 KB
            case 448: return launch_direct<7, 1, 2>(s, blocks, N, rowbytes, x, y, 1);
            case 512: return launch_digits<8, 1, 2, 2, 5>(s, blocks, N, rowbytes, x, y, 1);    // 2 rows, 34 KB
            default: break;
        }
    }
    return q8_dispatch<true>(s, blocks, 1, N, K, x, y);
}

}  // namespace aesir
