"""Shared helpers of the GPU quantized-weight tests: packed GGUF blocks of every type with weights
of a chosen spread, the f16 weights the library multiplies for them (from the oracle), and the
comparison rules."""
import numpy as np

F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 = 1, 2, 3, 6, 7, 8
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 10, 11, 12, 13, 14
LEGACY = {Q4_1: "q4_1", Q5_0: "q5_0", Q5_1: "q5_1"}
KQUANT = {Q2_K: "q2_k", Q3_K: "q3_k", Q5_K: "q5_k"}
NAMES = {Q4_0: "q4_0", Q4_1: "q4_1", Q5_0: "q5_0", Q5_1: "q5_1", Q8_0: "q8_0", Q2_K: "q2_k", Q3_K: "q3_k",
         Q4_K: "q4_k", Q5_K: "q5_k", Q6_K: "q6_k", F16: "f16"}
TYPE = {v: k for k, v in NAMES.items()}


def make_tensor(A, t, rows, cols, rng, std=0.02):
    """Packed blocks of GGML type t (or f16 values) for a rows x cols matrix of weights of spread
    near std."""
    if t == F16:
        return (rng.standard_normal((rows, cols)) * std).astype(np.float16)
    u = lambda shape: rng.uniform(0.5, 1.5, shape)
    nb, nsb = cols // 32, cols // 256
    if t == Q8_0:
        d = (u((rows, nb)) * std / 64).astype(np.float16)
        return A.Q8_0Tensor.from_parts(d, rng.integers(-127, 128, (rows, cols)).astype(np.int8))
    if t == Q4_0:
        d = (u((rows, nb)) * std / 4.6).astype(np.float16)
        return A.Q4_0Tensor.from_parts(d, rng.integers(0, 16, (rows, cols)).astype(np.uint8))
    if t in (Q4_1, Q5_0, Q5_1):
        top = 16 if t == Q4_1 else 32
        d = (u((rows, nb)) * std / (0.29 * top)).astype(np.float16)
        q = rng.integers(0, top, (rows, cols))
        if t == Q5_0:
            return A.Q5_0Tensor.from_parts(d, q)
        m = (-(top / 2 - 0.5 + rng.uniform(-1, 1, d.shape)) * d.astype(np.float64)).astype(np.float16)
        return (A.Q4_1Tensor if t == Q4_1 else A.Q5_1Tensor).from_parts(d, m, q)
    if t in (Q4_K, Q5_K):
        top = 16 if t == Q4_K else 32
        sc = rng.integers(1, 64, (rows, nsb, 8)).astype(np.uint8)
        mn = rng.integers(0, 64, (rows, nsb, 8)).astype(np.uint8)
        d = (u((rows, nsb)) * std / (32 * 0.29 * top)).astype(np.float16)
        dmin = (d.astype(np.float32) * rng.uniform(0.5, 1.0, (rows, nsb))).astype(np.float16)
        q = rng.integers(0, top, (rows, cols)).astype(np.uint8)
        return (A.Q4_KTensor if t == Q4_K else A.Q5_KTensor).from_parts(d, dmin, sc, mn, q)
    if t == Q6_K:
        sc = rng.integers(-127, 128, (rows, nsb, 16)).astype(np.int8)
        d = (u((rows, nsb)) * std / (64 * 18.5)).astype(np.float16)
        return A.Q6_KTensor.from_parts(d, sc, rng.integers(0, 64, (rows, cols)).astype(np.uint8))
    if t == Q2_K:
        d = (u((rows, nsb)) * std / (8 * 1.12)).astype(np.float16)
        dmin = (d.astype(np.float32) * rng.uniform(0.5, 1.0, (rows, nsb))).astype(np.float16)
        return A.Q2_KTensor.from_parts(d, dmin, rng.integers(1, 16, (rows, nsb, 16)), rng.integers(0, 16, (rows, nsb, 16)),
                                       rng.integers(0, 4, (rows, cols)))
    if t == Q3_K:
        d = (u((rows, nsb)) * std / (18.5 * 2.29)).astype(np.float16)
        return A.Q3_KTensor.from_parts(d, rng.integers(-32, 32, (rows, nsb, 16)), rng.integers(-4, 4, (rows, cols)))
    raise ValueError(f"type {t}")


def expected_f16(oracle, t, x):
    """The f16 weights [rows][cols] the library multiplies for tensor x of GGML type t."""
    if t == F16:
        return np.asarray(x, np.float16)
    nb = x.blocks.shape[0]
    if t == Q8_0:
        w = oracle.dequantize_q8_0(x.blocks, nb)
    elif t == Q4_0:
        w = oracle.dequantize_q4_0(x.blocks, nb)
    elif t in LEGACY:
        w = oracle.dequantize_legacy(LEGACY[t], x.blocks, nb)
    elif t in KQUANT:
        w = oracle.dequantize_kquant_f16(KQUANT[t], x.blocks, nb)
    elif t == Q4_K:
        w = oracle.dequantize_q4_k_f16(x.blocks, nb)
    else:
        w = oracle.dequantize_q6_k_f16(x.blocks, nb)
    return w.reshape(x.rows, x.cols)


def upload_bytes(ctx, raw):
    raw = np.ascontiguousarray(raw, np.uint8).reshape(-1)
    t = ctx.tensor(1, (raw.size + 1) // 2)
    buf = np.zeros(t.size * 2, np.uint8)
    buf[: raw.size] = raw
    t.upload(buf.view(np.float16))
    return t.ptr


def ulp_diff(a, b):
    ai = np.asarray(a, np.float16).view(np.int16).astype(np.int32)
    bi = np.asarray(b, np.float16).view(np.int16).astype(np.int32)
    ai = np.where(ai < 0, -32768 - ai, ai)
    bi = np.where(bi < 0, -32768 - bi, bi)
    return np.abs(ai - bi)


def same_token(got, want, ref_logits):
    """Equal tokens, or a near tie of the oracle's logits (within 2 f16 ulps)."""
    if got == want:
        return True
    a, b = float(ref_logits[got]), float(ref_logits[want])
    return abs(a - b) <= 2 * float(np.spacing(np.float16(max(abs(a), abs(b)))))


def within_tol(got, ref, atol=2e-2, rtol=1e-2):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return bool(np.all(np.abs(got - ref) <= atol + rtol * np.abs(ref)))
