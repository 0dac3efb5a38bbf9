"""GPU parity of the per-op kernels through the C ABI, against the CPU oracle on identical seeded
inputs (and, where the reference's own tests give one, the known answer).

Bars: bit-exact for integer/index work (argmax, KV copies, embedding) and for the elementwise
f16 ops whose arithmetic is fully determined (RoPE with the host-built table, SwiGLU product,
residual add, SiLU). Reductions in f32 (GEMV, RMSNorm's sum of squares) may differ from the
oracle's summation order by at most 1 f16 ulp. Attention keeps an f32 accumulator where the
reference stores f16 per position: max-abs 2e-2 / rel 1e-2 (the task tolerance).
"""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(1234)


@pytest.fixture(scope="module")
def A():
    import aesir_hip

    return aesir_hip


@pytest.fixture(scope="module")
def ctx(A):
    c = A.Context(4 << 30)
    print("device:", c.device_info(), flush=True)
    yield c
    c.close()


@pytest.fixture(autouse=True)
def well_scope(ctx):
    off = ctx.offset
    yield
    ctx.synchronize()
    ctx.reset(off)


def ulp_diff(a, b):
    ai = np.asarray(a, np.float16).view(np.int16).astype(np.int32)
    bi = np.asarray(b, np.float16).view(np.int16).astype(np.int32)
    ai = np.where(ai < 0, -32768 - ai, ai)
    bi = np.where(bi < 0, -32768 - bi, bi)
    return np.abs(ai - bi)


def within_tol(got, ref, atol=2e-2, rtol=1e-2):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return bool(np.all(np.abs(got - ref) <= atol + rtol * np.abs(ref)))


# ---------------------------------------------------------------- gemm_f16

def test_gemm_all_ones_32(A, ctx):
    """tests/test_compute.mojo:18-56."""
    a = ctx.from_numpy(np.ones((32, 32), np.float16))
    b = ctx.from_numpy(np.ones((32, 32), np.float16))
    c = ctx.tensor(32, 32)
    A.gemm_f16(ctx, a, b, c)
    assert np.all(c.numpy() == 32.0)


def test_gemm_rectangular_f32_reference(A, ctx, oracle):
    """tests/test_compute.mojo:315-357, plus the oracle to 1 ulp."""
    M, K, N = 17, 35, 29
    a_h = np.array([[np.float16((r + c) % 5 + 1) * np.float16(0.1) for c in range(K)] for r in range(M)], np.float16)
    b_h = np.array([[np.float16((r * c) % 7 + 1) * np.float16(0.1) for c in range(K)] for r in range(N)], np.float16)
    c = ctx.tensor(M, N)
    A.gemm_f16(ctx, ctx.from_numpy(a_h), ctx.from_numpy(b_h), c)
    got = c.numpy()
    assert np.max(np.abs(got.astype(np.float32) - a_h.astype(np.float32) @ b_h.astype(np.float32).T)) < 0.05
    assert np.max(ulp_diff(got, oracle.gemm_f16(a_h, b_h))) <= 1


@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (1, 4096, 1024), (1, 14336, 4096), (1, 4096, 28672),
                                   (1, 2048, 32000), (1, 64, 172), (1, 172, 64), (1, 35, 29), (3, 4096, 520),
                                   (1, 8, 1), (2, 4104, 33)])
def test_gemv_vs_oracle(A, ctx, oracle, M, K, N):
    """Micro-suite GEMV W ~ N(0, 0.02), x ~ N(0, 1): every output within 1 f16 ulp of the oracle."""
    x = RNG.standard_normal((M, K)).astype(np.float16)
    w = (RNG.standard_normal((N, K)) * 0.02).astype(np.float16)
    c = ctx.tensor(M, N)
    A.gemm_f16(ctx, ctx.from_numpy(x), ctx.from_numpy(w), c)
    got = c.numpy()
    ref = oracle.gemm_f16(x, w)
    d = ulp_diff(got, ref)
    # Beyond 1 ulp only where cancellation leaves a result so small that f32 summation-order noise
    # (bounded by 2^-17 of the sum of |products|) exceeds an f16 ulp.
    noise = 2.0 ** -17 * (np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T)
    bad = (d > 1) & (np.abs(got.astype(np.float64) - ref.astype(np.float64)) > noise)
    assert not bad.any(), (d.max(), np.argmax(d))
    assert (d > 0).mean() < 0.01


def test_gemm_errors(A, ctx):
    """compute.mojo:1756-1761, tests/test_compute.mojo:219-231."""
    a = ctx.tensor(2, 4)
    with pytest.raises(A.AesirError, match="inner matrix dimension mismatch"):
        A.gemm_f16(ctx, a, ctx.tensor(3, 8), ctx.tensor(2, 3))
    with pytest.raises(A.AesirError, match="output matrix shape mismatch"):
        A.gemm_f16(ctx, a, ctx.tensor(3, 4), ctx.tensor(2, 2))
    with pytest.raises(A.AesirError, match="dimensions must be positive"):
        A.gemm_f16(ctx, a.view(0, 4), ctx.tensor(3, 4), ctx.tensor(0, 3))


# ---------------------------------------------------------------- rmsnorm

@pytest.mark.parametrize("rows,cols", [(1, 4096), (64, 4096), (3, 35), (1, 64), (2, 14336)])
def test_rmsnorm_vs_oracle(A, ctx, oracle, rows, cols):
    x = RNG.standard_normal((rows, cols)).astype(np.float16)
    w = (1 + 0.1 * RNG.standard_normal(cols)).astype(np.float16)
    t = ctx.from_numpy(x)
    A.rmsnorm(ctx, t, ctx.from_numpy(w), 1e-5)
    got = t.numpy()
    ref = oracle.rmsnorm_f16(x, w, 1e-5)
    d = ulp_diff(got, ref)
    assert d.max() <= 1
    assert (d > 0).mean() < 0.01


def test_rmsnorm_constant_row_exact(A, ctx, oracle):
    x = np.full((4, 4096), 0.75, np.float16)
    w = RNG.standard_normal(4096).astype(np.float16)
    t = ctx.from_numpy(x)
    A.rmsnorm(ctx, t, ctx.from_numpy(w))
    assert np.array_equal(t.numpy().view(np.uint16), oracle.rmsnorm_f16(x, w).view(np.uint16))


def test_rmsnorm_errors(A, ctx):
    with pytest.raises(A.AesirError, match="weight dimension mismatch"):
        A.rmsnorm(ctx, ctx.tensor(2, 16), ctx.tensor(1, 8))
    with pytest.raises(A.AesirError, match="epsilon must be positive"):
        A.rmsnorm(ctx, ctx.tensor(1, 16), ctx.tensor(1, 16), 0.0)


# ---------------------------------------------------------------- rope

@pytest.mark.parametrize("rows,hd,nq,nk,start,theta", [
    (4096, 128, 32, 8, 0, 10000.0),      # micro-suite: Q [4096 x 32*128], K [4096 x 8*128], positions 0..4095
    (1, 128, 32, 8, 2047, 10000.0),
    (7, 64, 32, 4, 100000, 10000.0),     # grows the cached table
    (3, 8, 8, 4, 5, 500000.0),
])
def test_rope_bit_exact(A, ctx, oracle, rows, hd, nq, nk, start, theta):
    q = RNG.standard_normal((rows, nq * hd)).astype(np.float16)
    k = RNG.standard_normal((rows, nk * hd)).astype(np.float16)
    tq, tk = ctx.from_numpy(q), ctx.from_numpy(k)
    A.apply_rope(ctx, tq, tk, start, hd, theta)
    rq, rk = oracle.rope_f16(q, k, start, hd, theta)
    assert np.array_equal(tq.numpy().view(np.uint16), rq.view(np.uint16))
    assert np.array_equal(tk.numpy().view(np.uint16), rk.view(np.uint16))


def test_rope_errors(A, ctx):
    """tests/test_compute.mojo:247-256."""
    with pytest.raises(A.AesirError, match="head_dim must be positive and even"):
        A.apply_rope(ctx, ctx.tensor(1, 15), ctx.tensor(1, 15), 0, 15)
    with pytest.raises(A.AesirError, match="start_pos cannot be negative"):
        A.apply_rope(ctx, ctx.tensor(1, 16), ctx.tensor(1, 16), -1, 8)


# ---------------------------------------------------------------- attention

def attn_case(ctx, A, S, hd, nq, nkv, scale_kv=1.0):
    q = RNG.standard_normal((1, nq * hd)).astype(np.float16)
    K = (RNG.standard_normal((S, nkv * hd)) * scale_kv).astype(np.float16)
    V = RNG.standard_normal((S, nkv * hd)).astype(np.float16)
    out = ctx.tensor(1, nq * hd)
    A.flash_attention_gqa(ctx, ctx.from_numpy(q), ctx.from_numpy(K), ctx.from_numpy(V), out, S, hd, nq, nkv)
    return q, K, V, out.numpy()


def f64_attention(q, K, V, S, hd, nq, nkv):
    qd = q.astype(np.float64).reshape(nq, hd)
    Kd = K.astype(np.float64).reshape(S, nkv, hd)
    Vd = V.astype(np.float64).reshape(S, nkv, hd)
    g = np.arange(nq) // (nq // nkv)
    sc = np.einsum("hd,shd->hs", qd, Kd[:, g, :]) / math.sqrt(hd)
    p = np.exp(sc - sc.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    return np.einsum("hs,shd->hd", p, Vd[:, g, :]).reshape(-1)


def test_attention_uniform(A, ctx):
    """tests/test_compute.mojo:390-421."""
    q = ctx.from_numpy(np.full((1, 128), 0.1, np.float16))
    K = ctx.from_numpy(np.full((8, 32), 0.1, np.float16))
    V = ctx.from_numpy(np.full((8, 32), 0.3, np.float16))
    out = ctx.tensor(1, 128)
    A.flash_attention_gqa(ctx, q, K, V, out, 8, 16, 8, 2)
    assert np.all(np.abs(out.numpy().astype(np.float32) - 0.3) < 0.02)


def test_attention_single_position_maps_heads(A, ctx):
    """S = 1: head h returns V[h // (nq/nkv)] exactly (pins the GQA mapping)."""
    hd, nq, nkv = 128, 32, 8
    q, K, V, out = attn_case(ctx, A, 1, hd, nq, nkv)
    for h in range(nq):
        g = h // (nq // nkv)
        assert np.array_equal(out[0, h * hd:(h + 1) * hd], V[0, g * hd:(g + 1) * hd])


@pytest.mark.parametrize("S,hd,nq,nkv", [(37, 16, 8, 2), (80, 8, 8, 4), (512, 64, 32, 4), (2048, 128, 32, 8),
                                         (8192, 128, 32, 8), (200, 40, 4, 2), (65, 128, 32, 8),
                                         # register-resident path (head_dim 64/128): one split, a
                                         # partial last tile, ragged splits, 1/2/3/4/8 heads per KV
                                         # head, many tiles per split
                                         (31, 128, 32, 8), (33, 128, 32, 8), (2049, 128, 32, 8),
                                         (100, 128, 16, 8), (777, 64, 8, 8), (300, 64, 12, 4),
                                         (1000, 64, 32, 4), (4097, 64, 32, 4), (32768, 128, 32, 8),
                                         # views of 64 rounds and more (every split takes several
                                         # rounds): 4, 2 and 1 heads per KV head at head_dim 128
                                         # and 64, 3 heads per KV head, 65 rounds
                                         (4160, 128, 32, 8), (8192, 128, 16, 8), (5000, 128, 8, 8),
                                         (6000, 64, 16, 8), (5000, 64, 8, 8), (4500, 128, 24, 8),
                                         (20000, 64, 32, 4)])
def test_attention_vs_oracle_and_f64(A, ctx, oracle, S, hd, nq, nkv):
    q, K, V, out = attn_case(ctx, A, S, hd, nq, nkv)
    if S <= 8192:  # beyond this the reference's per-position f16 accumulator itself drifts
        ref_o = oracle.attn_gqa(q, K, V, np.zeros((1, nq * hd), np.float16), S, hd, nq, nkv)
        assert within_tol(out, ref_o)
    # the f32 accumulator is closer to the exact value than the reference's f16 accumulator
    assert within_tol(out[0], f64_attention(q, K, V, S, hd, nq, nkv), atol=2e-3, rtol=2e-3)


def test_attention_peaked_scores(A, ctx, oracle):
    """Large logits: the online softmax must rescale across tiles and splits correctly."""
    q, K, V, out = attn_case(ctx, A, 3000, 128, 32, 8, scale_kv=4.0)
    assert within_tol(out[0], f64_attention(q, K, V, 3000, 128, 32, 8), atol=2e-3, rtol=2e-3)


def test_attention_repeated_calls_varying_split_counts(A, ctx):
    """Back-to-back calls with shrinking and growing split counts (32, 1, 1, 11, 32, 1 splits of
    the head_dim 128 path) reuse the same partial buffer: each call's merge must read only its own
    splits' partials, and the single-split calls write the output without a merge."""
    hd, nq, nkv = 128, 32, 8
    for S in (2048, 40, 1, 700, 2048, 33):
        q, K, V, out = attn_case(ctx, A, S, hd, nq, nkv)
        assert within_tol(out[0], f64_attention(q, K, V, S, hd, nq, nkv), atol=2e-3, rtol=2e-3), S


def test_attention_alternating_long_and_short_views(A, ctx):
    """Views split 64 ways (one to three rounds a split), 33 ways and not at all alternate through
    one partial buffer: each merge must use its own call's split plan."""
    hd, nq, nkv = 128, 32, 8
    for S in (8192, 4096, 4097, 40, 12000, 2049, 4160):
        q, K, V, out = attn_case(ctx, A, S, hd, nq, nkv)
        assert within_tol(out[0], f64_attention(q, K, V, S, hd, nq, nkv), atol=2e-3, rtol=2e-3), S


@pytest.mark.parametrize("S,hd,nq,nkv", [(2048, 128, 32, 8), (3000, 64, 16, 4), (130, 128, 8, 8), (5000, 128, 32, 8)])
def test_attention_merge_sees_every_partial(A, ctx, S, hd, nq, nkv):
    """The split merge reads partials that the split workgroups wrote into the context's shared
    partial buffer. Two inputs alternate 60 times through the same buffers: every result must
    equal that input's first result bit for bit (a partial left over from the other input would
    change it), and the first results match f64."""
    cases = []
    for _ in range(2):
        q = RNG.standard_normal((1, nq * hd)).astype(np.float16)
        K = RNG.standard_normal((S, nkv * hd)).astype(np.float16)
        V = RNG.standard_normal((S, nkv * hd)).astype(np.float16)
        cases.append((q, K, V, ctx.from_numpy(q), ctx.from_numpy(K), ctx.from_numpy(V)))
    out = ctx.tensor(1, nq * hd)
    first = []
    for i in range(120):
        q, K, V, dq, dK, dV = cases[i % 2]
        A.flash_attention_gqa(ctx, dq, dK, dV, out, S, hd, nq, nkv)
        got = out.numpy()
        if i < 2:
            assert within_tol(got[0], f64_attention(q, K, V, S, hd, nq, nkv), atol=2e-3, rtol=2e-3)
            first.append(got.copy())
        else:
            assert np.array_equal(got.view(np.uint16), first[i % 2].view(np.uint16)), i


def test_attention_no_op_cases(A, ctx):
    """compute.mojo:1961-1966: output untouched."""
    q = ctx.from_numpy(np.full((1, 8), 0.5, np.float16))
    K = ctx.from_numpy(np.full((1, 8), 0.5, np.float16))
    base = np.zeros((1, 8), np.float16)
    base[0, 0] = 7.0
    for args in [(1, 0, 4, 2), (1, 4, 3, 2), (0, 4, 2, 2), (1, 4, 0, 1)]:
        out = ctx.from_numpy(base)
        A.flash_attention_gqa(ctx, q, K, K, out, *args)
        assert out.numpy()[0, 0] == 7.0


# ---------------------------------------------------------------- silu / swiglu / residual

def test_silu_all_f16_values(A, ctx, oracle):
    x = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    t = ctx.from_numpy(x.reshape(1, -1))
    A.silu(ctx, t)
    got = t.numpy().reshape(-1)
    ref = oracle.silu_f16(x)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint16), ref[~nan].view(np.uint16))


def test_silu_reference_kats(A, ctx):
    """tests/test_compute.mojo:102-131 and :359-388."""
    t = ctx.from_numpy(np.ones((1, 35), np.float16))
    A.silu(ctx, t)
    assert np.all(np.abs(t.numpy().astype(np.float32) - 0.7311) < 0.05)
    x = ((np.arange(37) - 18) * 0.25).astype(np.float32)
    t = ctx.from_numpy(x.astype(np.float16).reshape(1, -1))
    A.silu(ctx, t)
    assert np.max(np.abs(t.numpy()[0].astype(np.float32) - x / (1 + np.exp(-x)))) < 0.02


def test_swiglu_and_residual_exact(A, ctx, oracle):
    up = RNG.standard_normal(14336).astype(np.float16)
    gate = (RNG.standard_normal(14336) * 3).astype(np.float16)
    tu, tg = ctx.from_numpy(up), ctx.from_numpy(gate)
    A.swiglu(ctx, tu, tg)
    ref_gate = oracle.silu_f16(gate)
    assert np.array_equal(tg.numpy()[0].view(np.uint16), ref_gate.view(np.uint16))
    assert np.array_equal(tu.numpy()[0].view(np.uint16), oracle.mul_f16(up, ref_gate).view(np.uint16))
    x = RNG.standard_normal(4096).astype(np.float16)
    r = RNG.standard_normal(4096).astype(np.float16)
    tx = ctx.from_numpy(x)
    A.residual_add(ctx, tx, ctx.from_numpy(r))
    assert np.array_equal(tx.numpy()[0].view(np.uint16), oracle.residual_add_f16(x, r).view(np.uint16))


# ---------------------------------------------------------------- argmax / embedding / KV

def test_argmax_closed_forms(A, ctx, oracle):
    """inference.mojo:508-515: ties -> lowest index, floor -10000 -> 0, NaN skipped, +Inf wins."""
    cases = []
    x = np.zeros(128256, np.float16)
    x[77] = 3.0
    x[90000] = 3.0
    cases.append((x, 77))
    cases.append((np.full(100, -20000.0, np.float16), 0))
    y = np.full(5000, -20000.0, np.float16)
    y[4097] = -9992.0
    cases.append((y, 4097))
    z = np.zeros(3000, np.float16)
    z[3] = np.nan
    z[2049] = 1.0
    cases.append((z, 2049))
    z2 = z.copy()
    z2[2999] = np.inf
    cases.append((z2, 2999))
    t = np.zeros(128256, np.float16)  # planted ties on both sides of every group boundary
    t[[2047, 2048, 4095, 4096, 128255]] = 5.0
    cases.append((t, 2047))
    for arr, want in cases:
        assert A.argmax(ctx, ctx.from_numpy(arr)) == want == oracle.argmax_f16(arr)


@pytest.mark.parametrize("n", [1, 7, 512, 32000, 128256, 1000003])
def test_argmax_random_vs_oracle(A, ctx, oracle, n):
    x = RNG.standard_normal(n).astype(np.float16)  # f16 grid makes ties common: tests tie-break
    assert A.argmax(ctx, ctx.from_numpy(x)) == oracle.argmax_f16(x)


def test_embedding(A, ctx):
    table = RNG.standard_normal((512, 64)).astype(np.float16)
    t = ctx.from_numpy(table)
    x = ctx.tensor(1, 64)
    A.embed(ctx, t, 300, x)
    assert np.array_equal(x.numpy()[0], table[300])
    with pytest.raises(A.AesirError, match="outside the embedding vocabulary"):
        A.embed(ctx, t, 512, x)


def test_kv_cache_known_answers(A, ctx):
    """tests/test_kv_cache.mojo:32-50 and :114-129, with the ring slot pos % max_seq."""
    kv = A.KVCache(ctx, 64, 16, 2)
    k = ctx.from_numpy(np.arange(1, 17, dtype=np.float16))
    v = ctx.from_numpy((2 * np.arange(1, 17)).astype(np.float16))
    kv.append(0, 0, k, v)
    assert kv.get_k_slice(0, 1).numpy()[0, 0] == 1.0 and kv.get_v_slice(0, 1).numpy()[0, 0] == 2.0
    kv.append(1, 64 + 5, v, k)
    ks = kv.get_k_slice(1, 64).numpy()
    assert np.array_equal(ks[5], (2 * np.arange(1, 17)).astype(np.float16))
    with pytest.raises(A.AesirError, match="layer_idx out of bounds"):
        kv.get_k_slice(10, 1)
    with pytest.raises(A.AesirError, match="seq_len out of bounds"):
        kv.get_v_slice(0, 500)
    with pytest.raises(A.AesirError, match="width mismatch"):
        kv.append(0, 0, k.view(1, 8), v)


def test_well_exhaustion(A):
    """tests/test_kv_cache.mojo:88-99: MimirWell raises on exhaustion."""
    with A.Context(1024) as small:
        with pytest.raises(A.AesirError, match="MimirWell: memory pool exhausted"):
            small.allocate(1000)
        off = small.offset
        small.allocate(100)
        small.reset(off)
        assert small.offset == off
        with pytest.raises(A.AesirError, match="invalid reset offset"):
            small.reset(off + 10**6)


# ---------------------------------------------------------------- Q8_0

def make_q8_0(n_rows, K, rng):
    nb = n_rows * K // 32
    d = rng.uniform(0.001, 0.02, nb).astype(np.float16)
    q = rng.integers(-127, 128, (nb, 32)).astype(np.int8)
    blocks = np.zeros((nb, 34), np.uint8)
    blocks[:, :2] = d.view(np.uint8).reshape(nb, 2)
    blocks[:, 2:] = q.view(np.uint8)
    return blocks, d, q


def upload_bytes(ctx, raw: np.ndarray) -> int:
    raw = np.ascontiguousarray(raw, np.uint8).reshape(-1)
    t = ctx.tensor(1, (raw.size + 1) // 2)
    buf = np.zeros(t.size * 2, np.uint8)
    buf[: raw.size] = raw
    t.upload(buf.view(np.float16))
    return t.ptr


@pytest.mark.parametrize("N,K", [(48, 256), (64, 4096), (33, 96), (50, 512), (37, 16384), (5, 32768)])
def test_gemm_q8_0_vs_oracle(A, ctx, oracle, N, K):
    """Rows of K / 32 blocks with (K / 32) % 8 == 0 are staged through LDS, 4, 2 or 1 rows per
    workgroup by row length (K = 256 .. 14336: 4; 16384: 2; 32768: 1), including a last workgroup
    with fewer rows (N = 50, 37, 5); K = 96 takes the per-lane block-pair kernel."""
    blocks, d, q = make_q8_0(N, K, RNG)
    a = RNG.standard_normal((1, K)).astype(np.float16)
    c = ctx.tensor(1, N)
    A.gemm_q8_0(ctx, ctx.from_numpy(a), upload_bytes(ctx, blocks), N, c)
    got = c.numpy()
    ref = oracle.gemm_q8_0(a, blocks, N)
    # Beyond 1 ulp only where the result is small enough that f32 summation-order noise (bounded
    # by 2^-17 of the sum of |products|) exceeds an f16 ulp.
    W = oracle.dequantize_q8_0(blocks, N * K // 32).reshape(N, K).astype(np.float64)
    noise = 2.0 ** -17 * (np.abs(a.astype(np.float64)) @ np.abs(W).T)
    d = ulp_diff(got, ref)
    bad = (d > 1) & (np.abs(got.astype(np.float64) - ref.astype(np.float64)) > noise)
    assert not bad.any(), (d.max(), np.argwhere(bad)[:4])
    assert (d > 0).mean() < 0.1


@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336), (37, 16384), (29, 96), (4100, 2048), (2050, 8192),
                                 (600, 16384), (3, 14336), (50, 512)])
def test_q8_0_matvec_f32_closed_form(A, ctx, N, K):
    """Config 5: fp32 dequantize-then-matvec of the same blocks (closed form, f64). Rows of 64, 128,
    256, 448 and 512 blocks take the integer-digit kernel (more row groups than workgroups, and a
    last group with fewer rows: 4100, 2050, 600); 16 and 3 blocks the staged and pair kernels."""
    blocks, d, q = make_q8_0(N, K, RNG)
    x = RNG.standard_normal(K).astype(np.float32)
    y = ctx.tensor(1, N, np.float32)
    A.q8_0_matvec_f32(ctx, upload_bytes(ctx, blocks), N, K, ctx.from_numpy(x, np.float32), y)
    W = (q.astype(np.float64) * d.astype(np.float64)[:, None]).reshape(N, K)
    ref = W @ x.astype(np.float64)
    got = y.numpy()[0].astype(np.float64)
    # f32 arithmetic: error bounded by 2^-17 of the sum of |products|
    noise = 2.0 ** -17 * (np.abs(W) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(got - ref) <= noise)


@pytest.mark.parametrize("K", [2048, 4096, 14336, 16384])
def test_q8_0_matvec_f32_outlier_blocks(A, ctx, K):
    """Activations with outlier channels: every block holds 1000 beside N(0, 1e-3) values and the
    outlier's quant is 0, so the small values carry the dot product. The GPU equals the sum of the
    emulated digit-kernel block values (q8_digits.py) up to f32 summation over blocks, and stays
    within the stated bound of the exact f64 result: 2^-30 * max|x_blk| * sum|d q| per block plus
    f32 rounding and summation."""
    from q8_digits import block_bound, block_values

    N, nb = 96, K // 32
    blocks, d, q = make_q8_0(N, K, RNG)
    x = (RNG.standard_normal(K) * 1e-3).astype(np.float32)
    x[::32] = 1000.0
    q = q.reshape(N, nb, 32).copy()
    q[:, :, 0] = 0
    blocks[:, 2:] = q.reshape(-1, 32).view(np.uint8)
    y = ctx.tensor(1, N, np.float32)
    A.q8_0_matvec_f32(ctx, upload_bytes(ctx, blocks), N, K, ctx.from_numpy(x, np.float32), y)
    got = y.numpy()[0].astype(np.float64)
    dd = d.reshape(N, nb)
    emu = block_values(x.reshape(nb, 32), q, dd).astype(np.float64)
    sum_noise = 2.0 ** -20 * np.abs(emu).sum(axis=1)
    assert np.all(np.abs(got - emu.sum(axis=1)) <= sum_noise)
    exact = (q.astype(np.float64) * dd.astype(np.float64)[:, :, None]).reshape(N, K) @ x.astype(np.float64)
    assert np.all(np.abs(got - exact) <= block_bound(x.reshape(nb, 32), q, dd).sum(axis=1) + sum_noise)


@pytest.mark.parametrize("K", [4096, 14336])
def test_q8_0_matvec_f32_non_finite_x(A, ctx, K):
    """An inf in x reaches every row as in the f32 formula (+-inf, or NaN where 0 * inf or inf - inf
    occurs); the other blocks of the row keep their digit path."""
    N = 96
    blocks, d, q = make_q8_0(N, K, RNG)
    x = RNG.standard_normal(K).astype(np.float32)
    x[5] = np.inf
    x[K - 40] = -np.inf
    y = ctx.tensor(1, N, np.float32)
    A.q8_0_matvec_f32(ctx, upload_bytes(ctx, blocks), N, K, ctx.from_numpy(x, np.float32), y)
    W = (q.astype(np.float64) * d.astype(np.float64)[:, None]).reshape(N, K)
    with np.errstate(invalid="ignore"):
        ref = W @ x.astype(np.float64)
    got = y.numpy()[0].astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    x[5] = np.nan
    A.q8_0_matvec_f32(ctx, upload_bytes(ctx, blocks), N, K, ctx.from_numpy(x, np.float32), y)
    assert np.isnan(y.numpy()).all()
