"""GPU parity of the repacked weight types, Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q4_K, Q5_K and Q6_K
(tiled records, the matrix-core decode GEMV with the fused epilogues, batched prefill, GGUF
loading), against the CPU oracle.

- aesir_gemm_quant on packed GGUF blocks: Q4_0, Q4_1, Q5_0 and Q5_1 within 1 f16 ulp of the
  oracle's reference-order gemm_q4_0 / _q4_1 / _q5_0 / _q5_1 (core/compute.mojo:876-1036; beyond
  1 ulp only where f32 summation noise exceeds it); the K-quants against f64 on the oracle's
  f16 weights (the rule every kernel of the library applies) within one f16 rounding of the
  output plus f32 summation noise. 16 or more rows of A, and rows whose length is not a multiple
  of 128, take the F16 GEMM on the same f16 weights and are held to f64 on those.
- Models: the F16 oracle holding the weights the model reads back (get_tensor), which are the
  f16 weights the GEMVs and the prefill multiply for every type; Q4_0 tokens are identical, the
  others may differ only at a near tie of the oracle's logits, and logits are held to the
  forward-pass tolerance.
"""
import numpy as np
import pytest

from quant_tools import expected_f16, make_tensor, same_token, ulp_diff, upload_bytes, within_tol

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(4321)


@pytest.fixture(scope="module")
def A():
    import aesir_hip

    return aesir_hip


@pytest.fixture(scope="module")
def ctx(A):
    c = A.Context(3 << 30)
    yield c
    c.close()


@pytest.fixture(autouse=True)
def well_scope(ctx):
    off = ctx.offset
    yield
    ctx.synchronize()
    ctx.reset(off)


TYPES = {"q4_0": 2, "q4_1": 3, "q5_0": 6, "q5_1": 7, "q2_k": 10, "q3_k": 11, "q4_k": 12, "q5_k": 13, "q6_k": 14}
LEGACY_KINDS = ("q4_1", "q5_0", "q5_1")


def random_tensor(A, kind, rows, cols, rng, std=0.02):
    """Packed GGUF blocks of a rows x cols matrix with weights of standard deviation near std."""
    return make_tensor(A, TYPES[kind], rows, cols, rng, std)


def lib_weights(oracle, kind, t):
    """The f16 weights the library multiplies, as f64."""
    return expected_f16(oracle, TYPES[kind], t).astype(np.float64)


@pytest.mark.parametrize("kind", list(TYPES))
@pytest.mark.parametrize("M,K,N", [(1, 4096, 64), (1, 14336, 40), (3, 2048, 100), (1, 5632, 33), (1, 28672, 8),
                                   (20, 4096, 48), (1, 512, 16400), (2, 1536, 18000), (128, 2048, 96),
                                   (100, 4096, 200), (128, 1024, 5000)])
def test_gemm_quant_vs_oracle(A, ctx, oracle, kind, M, K, N):
    """M < 16: the decode GEMV per row on the repacked planes; M > 64: the wide-tile matrix-core
    GEMM on the same planes (K splits with a reduce, M and N tails, 64- and 32-column tiles);
    otherwise the F16 GEMM on dequantized weights."""
    t = random_tensor(A, kind, N, K, RNG)
    x = RNG.standard_normal((M, K)).astype(np.float16)
    c = ctx.tensor(M, N)
    A.gemm_quant(ctx, ctx.from_numpy(x), upload_bytes(ctx, t.blocks), TYPES[kind], N, c)
    got = c.numpy().astype(np.float64)
    W = lib_weights(oracle, kind, t)
    xd = x.astype(np.float64)
    noise = 2.0 ** -17 * (np.abs(xd) @ np.abs(W).T)
    if kind in ("q4_0",) + LEGACY_KINDS and M < 16:
        ref = oracle.gemm_q4_0(x, t.blocks, N) if kind == "q4_0" else oracle.gemm_legacy(kind, x, t.blocks, N)
        d = ulp_diff(got.astype(np.float16), ref)
        bad = (d > 1) & (np.abs(got - ref.astype(np.float64)) > noise)
        assert not bad.any(), d.max()
        assert (d > 0).mean() < 0.02 or (d > 0).sum() <= 1  # nearly all outputs identical
        return
    exact = xd @ W.T
    tol = np.abs(np.spacing(exact.astype(np.float16))).astype(np.float64) + noise
    assert np.all(np.abs(got - exact) <= tol), np.max(np.abs(got - exact) / tol)


@pytest.mark.parametrize("kind", ("q4_0",) + LEGACY_KINDS)
@pytest.mark.parametrize("M,K,N", [(1, 160, 24), (3, 96, 40), (1, 28704, 17)])
def test_gemm_q4_0_rows_off_the_tile_grid(A, ctx, oracle, kind, M, K, N):
    """Rows of the 32-weight block types whose length is not a multiple of 128 (or above the GEMV's
    28672) take the f16 dequantization + F16 GEMM route: within 1 f16 ulp of the oracle's
    reference-order gemm_q4_0 / _q4_1 / _q5_0 / _q5_1 where f32 summation noise does not exceed it."""
    t = random_tensor(A, kind, N, K, RNG)
    x = RNG.standard_normal((M, K)).astype(np.float16)
    c = ctx.tensor(M, N)
    A.gemm_quant(ctx, ctx.from_numpy(x), upload_bytes(ctx, t.blocks), TYPES[kind], N, c)
    got = c.numpy()
    ref = oracle.gemm_q4_0(x, t.blocks, N) if kind == "q4_0" else oracle.gemm_legacy(kind, x, t.blocks, N)
    W = lib_weights(oracle, kind, t)
    noise = 2.0 ** -17 * (np.abs(x.astype(np.float64)) @ np.abs(W).T)
    d = ulp_diff(got, ref)
    assert not ((d > 1) & (np.abs(got.astype(np.float64) - ref.astype(np.float64)) > noise)).any(), d.max()


@pytest.mark.parametrize("kind", ("q4_0", "q4_k", "q6_k"))
@pytest.mark.parametrize("M", (1, 100))
def test_gemm_quant_unaligned_a(A, ctx, oracle, kind, M):
    """A as an offset view (2-byte aligned, not 16-byte): the repacked-plane routes need 16-byte
    loads of A, so the call takes the dequantize-then-F16 route at 1 row (the GEMV's) and at 100
    rows (the wide kernel's) and still matches f64 on the library's f16 weights."""
    K, N = 4096, 96
    t = random_tensor(A, kind, N, K, RNG)
    x = RNG.standard_normal((M, K)).astype(np.float16)
    buf = ctx.from_numpy(np.concatenate([np.zeros(1, np.float16), x.reshape(-1)]).reshape(1, -1))
    a = buf.view(M, K, offset_elems=1)
    assert a.ptr % 16 != 0
    c = ctx.tensor(M, N)
    A.gemm_quant(ctx, a, upload_bytes(ctx, t.blocks), TYPES[kind], N, c)
    got = c.numpy().astype(np.float64)
    W = lib_weights(oracle, kind, t)
    xd = x.astype(np.float64)
    exact = xd @ W.T
    tol = np.abs(np.spacing(exact.astype(np.float16))).astype(np.float64) + 2.0 ** -17 * (np.abs(xd) @ np.abs(W).T)
    assert np.all(np.abs(got - exact) <= tol), np.max(np.abs(got - exact) / tol)


def test_gemm_quant_errors(A, ctx):
    a = ctx.tensor(1, 96)
    c = ctx.tensor(1, 2)
    with pytest.raises(A.AesirError, match="gemm_q4_0: inner dimension must be a multiple of 32"):
        A.gemm_quant(ctx, ctx.tensor(1, 40), a.ptr, 2, 2, c)
    with pytest.raises(A.AesirError, match="gemm_q4_k: inner dimension must be a multiple of 256"):
        A.gemm_quant(ctx, a, a.ptr, 12, 2, c)
    with pytest.raises(A.AesirError, match="gemm_q6_k: output matrix shape mismatch"):
        A.gemm_quant(ctx, ctx.tensor(1, 256), a.ptr, 14, 3, c)
    with pytest.raises(A.AesirError, match="is not Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K or Q6_K"):
        A.gemm_quant(ctx, a, a.ptr, 9, 2, c)
    with pytest.raises(A.AesirError, match="gemm_q5_k: inner dimension must be a multiple of 256"):
        A.gemm_quant(ctx, a, a.ptr, 13, 2, c)


def quant_weights(A, oracle, cfg, kind, rng):
    w = {}
    for name, (r, c) in oracle.tensor_shapes(cfg).items():
        if name.endswith("norm.weight"):
            w[name] = (1.0 + 0.05 * rng.standard_normal(c)).astype(np.float16)
        else:
            w[name] = random_tensor(A, kind, r, c, rng)
    return w


def quant_model(A, ctx, oracle, cfg, kind, seed):
    rng = np.random.default_rng(seed)
    m = A.Model.create(ctx, A.ModelConfig(cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.ffn, cfg.vocab,
                                          cfg.ctx_len, cfg.eps, cfg.theta, 1, -1), TYPES[kind])
    m.set_weights(quant_weights(A, oracle, cfg, kind, rng))
    back = {name: m.get_tensor(name, shape) for name, shape in oracle.tensor_shapes(cfg).items()}
    return m, oracle.Model(cfg, back)


SMALL = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, ffn=512, vocab=300, ctx_len=160)


@pytest.mark.parametrize("kind", list(TYPES))
def test_quant_model_stream_matches_dequantized_oracle(A, ctx, oracle, kind):
    """Per-position forward passes, then graph-replayed decode, against the F16 oracle on the
    read-back weights; graph replay == eager launches == the host loop."""
    cfg = oracle.Config(**SMALL)
    m, om = quant_model(A, ctx, oracle, cfg, kind, 5)
    prompt = oracle.prompt_tokens(12, cfg.vocab, 3)
    okv = om.new_kv()
    cur = list(prompt)
    for p in range(len(prompt) + 20):
        want, ol = om.forward(okv, cur, p)
        got = m.forward_pass(cur, p)
        assert within_tol(m.logits(), ol), (kind, p)
        if kind == "q4_0":
            assert got == want, p
        else:
            assert same_token(got, want, ol), (p, got, want)
        if p >= len(prompt) - 1:
            cur.append(got)
    nxt = cur[len(prompt)]
    g, _ = m.decode_loop(nxt, len(prompt), 16, use_graph=True)
    e, _ = m.decode_loop(nxt, len(prompt), 16, use_graph=False)
    host = []
    c2 = list(prompt) + [nxt]
    for _ in range(16):
        host.append(m.forward_pass(c2, len(c2) - 1))
        c2.append(host[-1])
    assert g == e == host
    m.close()


@pytest.mark.parametrize("kind", list(TYPES))
def test_quant_long_chunk_prefill_matches_per_position(A, ctx, oracle, kind):
    """A 300-row chunk: every GEMM dequantizes its matrix into the f16 copy (the type's own
    rounding) and runs on hipBLASLt, attention on the matrix-core kernel; next token (near ties
    allowed) and logits against the per-position oracle on the read-back weights."""
    cfg = oracle.Config(**{**SMALL, "ctx_len": 320})
    m, om = quant_model(A, ctx, oracle, cfg, kind, 7)
    prompt = oracle.prompt_tokens(300, cfg.vocab, 5)
    okv = om.new_kv()
    for p in range(len(prompt)):
        want, ol = om.forward(okv, prompt, p)
    got = m.prefill(prompt, 0)
    assert within_tol(m.logits(), ol)
    assert same_token(got, want, ol), (got, want)
    m.close()


@pytest.mark.parametrize("kind", list(TYPES))
def test_quant_batched_prefill_matches_per_position(A, ctx, oracle, kind):
    """aesir_prefill of a 140-token prompt (one chunk: two 128-row M tiles of the matrix-core GEMM on
    the repacked planes), and of the same prompt as 100 + 40 positions (the 40-row chunk on f16
    copies of the weights and 32-row tiles), against the per-position oracle: next token (near
    ties allowed) and logits within tolerance."""
    cfg = oracle.Config(**SMALL)
    m, om = quant_model(A, ctx, oracle, cfg, kind, 6)
    prompt = oracle.prompt_tokens(140, cfg.vocab, 4)
    okv = om.new_kv()
    for p in range(len(prompt)):
        want, ol = om.forward(okv, prompt, p)
    got = m.prefill(prompt, 0)
    assert within_tol(m.logits(), ol)
    assert same_token(got, want, ol), (got, want)
    m.close()
    m2, _ = quant_model(A, ctx, oracle, cfg, kind, 6)
    m2.prefill(prompt[:100], 0)
    got2 = m2.prefill(prompt[100:], 100)
    assert within_tol(m2.logits(), ol)
    assert same_token(got2, want, ol), (got2, want)
    m2.close()


@pytest.mark.parametrize("kind", list(TYPES))
def test_quant_gguf_file_loads_like_set_tensor(A, ctx, oracle, kind, tmp_path):
    """A GGUF file whose matrices are all of the type (norms F32) loads into the same model."""
    from gguf_tools import llama_metadata, write_gguf

    cfg = oracle.Config(**SMALL)
    rng = np.random.default_rng(7)
    w = quant_weights(A, oracle, cfg, kind, rng)
    tensors = {k: (v.astype(np.float32) if k.endswith("norm.weight") else v) for k, v in w.items()}
    path = str(tmp_path / f"{kind}.gguf")
    write_gguf(path, llama_metadata(cfg, cfg.vocab), tensors)
    mf = A.Model.load_gguf(ctx, path, cfg.ctx_len)
    assert mf.weight_type == TYPES[kind]
    ms = A.Model.create(ctx, A.ModelConfig(cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.ffn, cfg.vocab,
                                           cfg.ctx_len, cfg.eps, cfg.theta, 1, 2), TYPES[kind])
    ms.set_weights(w)
    prompt = oracle.prompt_tokens(6, cfg.vocab, 8)
    a, _ = mf.generate(prompt, 8)
    b, _ = ms.generate(prompt, 8)
    assert a == b
    name = "blk.1.ffn_down.weight"
    assert np.array_equal(mf.get_tensor(name, (cfg.dim, cfg.ffn)), ms.get_tensor(name, (cfg.dim, cfg.ffn)))
    mf.close()
    ms.close()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("kind", list(TYPES))
def test_quant_llama3_8b_shape_properties(A, oracle, kind):
    """Llama-3-8B shape with device-initialized weights of the type: graph == eager == forward_pass
    for 6 steps from KV 2048, finite logits, and the read-back of a matrix within its weight range."""
    cfg = oracle.LLAMA3_8B
    with A.Context(14 << 30) as big:
        m = A.Model.create(big, A.ModelConfig(cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.ffn, cfg.vocab,
                                              2048 + 16), TYPES[kind])
        m.init_random(11)
        m.fill_kv_random(2048, seed=2)
        g, _ = m.decode_loop(77, 2048, 6, use_graph=True)
        e, _ = m.decode_loop(77, 2048, 6, use_graph=False)
        cur = [0] * 2048 + [77]
        host = []
        for _ in range(6):
            host.append(m.forward_pass(cur, len(cur) - 1))
            assert np.all(np.isfinite(m.logits().astype(np.float32)))
            cur.append(host[-1])
        assert g == e == host
        wd = m.get_tensor("blk.0.ffn_down.weight", (cfg.dim, cfg.ffn)).astype(np.float32)
        assert np.isfinite(wd).all() and 0.01 < wd.std() < 0.04, wd.std()
        m.close()
