"""CPU emulation of the integer-digit Q8_0 matvec (q8_0_digits_kernel): the value each thread
computes for one (row, block). It is exact integer arithmetic plus the kernel's two roundings,
so the tests can check the kernel's stated error bound on adversarial blocks and compare the GPU
against the sum of these block values.

Per block: e = ilogb(max |x|); v_i = rint(x_i * 2^(29 - e)) (|v_i| <= 2^30); S = sum_i q_i v_i
(exact; the kernel forms it from four signed 8-bit digits of v with v_dot4_i32_i8); block value =
f32(ldexp(f64(S) * f64(d), e - 29))."""
import numpy as np


def block_values(x: np.ndarray, q: np.ndarray, d: np.ndarray) -> np.ndarray:
    """x: f32 [nb, 32]; q: int8 [rows, nb, 32]; d: f16 [rows, nb] -> f32 [rows, nb]."""
    x = np.asarray(x, np.float32)
    m = np.abs(x).max(axis=1)
    e = np.where(m > 0, np.frexp(m)[1] - 1, 0).astype(np.int64)  # ilogb
    v = np.rint(np.ldexp(x.astype(np.float64), (29 - e)[:, None])).astype(np.int64)  # exact scaling
    assert np.abs(v).max(initial=0) <= 1 << 30
    # the four signed digits, as the kernel splits them, recombine to v exactly
    d0 = ((v & 0xFF) ^ 0x80) - 0x80
    r1 = (v - d0) >> 8
    d1 = ((r1 & 0xFF) ^ 0x80) - 0x80
    r2 = (r1 - d1) >> 8
    d2 = ((r2 & 0xFF) ^ 0x80) - 0x80
    d3 = (r2 - d2) >> 8
    assert np.array_equal(d0 + (d1 << 8) + (d2 << 16) + (d3 << 24), v) and np.abs(d3).max(initial=0) <= 64
    S = np.einsum("rbi,bi->rb", q.astype(np.int64), v)
    assert np.abs(S).max(initial=0) < 1 << 44
    prod = S.astype(np.float64) * d.astype(np.float64)  # one f64 rounding
    return np.ldexp(prod, (e - 29)[None, :]).astype(np.float32)


def block_bound(x: np.ndarray, q: np.ndarray, d: np.ndarray) -> np.ndarray:
    """Stated per-block error bound: 2^-30 * max|x_blk| * sum|d q| plus the f32 rounding of the
    block value (2^-24 relative, taken on the exact value plus that term, or half the smallest
    f32 denormal, 2^-150, for results in the denormal range)."""
    m = np.abs(np.asarray(x, np.float64)).max(axis=1)
    sw = np.abs(q.astype(np.float64)).sum(axis=2) * np.abs(d.astype(np.float64))
    exact = np.einsum("rbi,bi->rb", q.astype(np.float64), np.asarray(x, np.float64)) * d.astype(np.float64)
    t = 2.0 ** -30 * m[None, :] * sw
    return t + 2.0 ** -24 * (np.abs(exact) + t) + 2.0 ** -150
