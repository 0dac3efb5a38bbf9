"""GPU parity of the batched prefill (aesir_prefill) and of the MFMA GEMM, against the CPU oracle.

- gemm_f16 with 16 or more rows of A runs on the MFMA kernel (v_mfma_f32_16x16x32_f16, f32
  accumulate): every output within 1 f16 ulp of the oracle's f32-accumulated gemm_f16 (more only
  where cancellation puts the result below f32 summation-order noise), fewer than 1% of outputs
  differing at all, including M and N tails and more than one 128-row tile.
- aesir_prefill over n prompt positions equals the reference's prefill by position
  (aesir.mojo:358-374, one forward_pass per position): the same next token, logits within
  max-abs 2e-2 / rel 1e-2, and the greedy decode that follows reads the K/V cache the prefill
  wrote and continues with the oracle's tokens. Covered: the tiny model (non-MFMA shapes: ffn 172),
  prompts longer than one 128-row chunk, continuation at start_pos > 0, the TinyLlama shape
  (MFMA GEMMs with the store, residual and SwiGLU epilogues) and the GQA-grouped attention tiles.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(4321)


@pytest.fixture(scope="module")
def A():
    import aesir_hip

    return aesir_hip


@pytest.fixture(scope="module")
def ctx(A):
    c = A.Context(4 << 30)
    yield c
    c.close()


@pytest.fixture(autouse=True)
def well_scope(ctx):
    off = ctx.offset
    yield
    ctx.synchronize()
    ctx.reset(off)


def within_tol(got, ref, atol=2e-2, rtol=1e-2):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return bool(np.all(np.abs(got - ref) <= atol + rtol * np.abs(ref)))


def ulp_diff(a, b):
    ai = np.asarray(a, np.float16).view(np.int16).astype(np.int32)
    bi = np.asarray(b, np.float16).view(np.int16).astype(np.int32)
    ai = np.where(ai < 0, -32768 - ai, ai)
    bi = np.where(bi < 0, -32768 - bi, bi)
    return np.abs(ai - bi)


def gpu_model(A, ctx, ocfg, weights):
    cfg = A.ModelConfig(ocfg.dim, ocfg.n_layers, ocfg.n_heads, ocfg.n_kv_heads, ocfg.ffn, ocfg.vocab, ocfg.ctx_len,
                        ocfg.eps, ocfg.theta, 1, -1)
    m = A.Model.create(ctx, cfg)
    m.set_weights(weights)
    return m


@pytest.mark.parametrize("M,K,N", [(16, 64, 32), (37, 4096, 1000), (128, 2048, 2560), (200, 256, 300),
                                   (128, 5632, 128), (129, 32, 17), (128, 2048, 11264), (100, 1024, 16500),
                                   (64, 128, 16384), (200, 256, 9000), (96, 8192, 256), (65, 384, 4100),
                                   (128, 4096, 1000), (2, 4096, 4096), (8, 2048, 5632), (15, 14336, 512)])
def test_mfma_gemm_vs_oracle(A, ctx, oracle, M, K, N):
    """The 32 x 64 kernel (M <= 64 or K % 128 != 0; from M = 2, rows past M read as zeros) and the
    128-row wide-tile kernel (M > 64,
    K % 128 == 0): NT = 64 columns from N = 4096 up, else 32; with M and N tails, a single K
    chunk, two M tiles, 8 K splits (96 x 8192 x 256, 128 x 4096 x 1000; fewer where the context's
    partial buffer is smaller) and an odd 3-chunk K without split (65 x 384 x 4100)."""
    a = RNG.standard_normal((M, K)).astype(np.float16)
    b = (RNG.standard_normal((N, K)) * 0.02).astype(np.float16)
    c = ctx.tensor(M, N)
    A.gemm_f16(ctx, ctx.from_numpy(a), ctx.from_numpy(b), c)
    got = c.numpy()
    want = oracle.gemm_f16(a, b)
    d = ulp_diff(got, want)
    # Beyond 1 ulp only where cancellation leaves a result so small that f32 summation-order noise
    # (bounded by 2^-17 of the sum of |products|) exceeds an f16 ulp.
    noise = 2.0 ** -17 * (np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64)).T)
    bad = (d > 1) & (np.abs(got.astype(np.float64) - want.astype(np.float64)) > noise)
    assert not bad.any(), (d.max(), np.argwhere(bad)[:4])
    assert (d > 0).mean() < 0.01


def oracle_prefill(om, prompt, n_extra=0):
    """Per-position forward over the prompt (the reference's prefill), then n_extra greedy steps."""
    kv = om.new_kv()
    cur = list(prompt)
    nxt, logits = None, None
    for p in range(len(prompt)):
        nxt, logits = om.forward(kv, cur, p)
    first_logits = logits
    follow = []
    for _ in range(n_extra):
        cur.append(nxt)
        follow.append(nxt)
        nxt, _ = om.forward(kv, cur, len(cur) - 1)
    return follow[0] if follow else nxt, first_logits, follow


def gpu_follow(m, prompt, first, n_extra):
    cur = list(prompt) + [first]
    out = [first]
    for _ in range(n_extra - 1):
        nxt = m.forward_pass(cur, len(cur) - 1)
        cur.append(nxt)
        out.append(nxt)
    return out


def test_prefill_tiny_matches_per_position(A, ctx, oracle):
    cfg = oracle.TINY
    w = oracle.synthetic_weights(cfg, 1234)
    om = oracle.Model(cfg, w)
    prompt = oracle.prompt_tokens(16, cfg.vocab, 7)
    first, ologits, follow = oracle_prefill(om, prompt, 8)
    m = gpu_model(A, ctx, cfg, w)
    got = m.prefill(prompt)
    assert within_tol(m.logits(), ologits)
    assert got == first
    assert gpu_follow(m, prompt, got, 8) == follow
    m.close()


def test_prefill_chunks_and_continuation(A, ctx, oracle):
    """2200 positions = 2048-row chunks 2048 + 152; then the same prompt as 100 + 2100 positions
    (start_pos 100: chunks 2048 + 52): both equal the per-position prefill."""
    import dataclasses

    cfg = dataclasses.replace(oracle.TINY, ctx_len=2300)
    w = oracle.synthetic_weights(cfg, 99)
    om = oracle.Model(cfg, w)
    prompt = oracle.prompt_tokens(2200, cfg.vocab, 11)
    first, ologits, follow = oracle_prefill(om, prompt, 4)
    m = gpu_model(A, ctx, cfg, w)
    got = m.prefill(prompt)
    assert within_tol(m.logits(), ologits)
    assert got == first
    assert gpu_follow(m, prompt, got, 4) == follow
    m.close()
    m2 = gpu_model(A, ctx, cfg, w)
    m2.prefill(prompt[:100])
    got2 = m2.prefill(prompt[100:], start_pos=100)
    assert within_tol(m2.logits(), ologits)
    assert got2 == first
    m2.close()


def test_prefill_tinyllama_shape_mfma(A, ctx, oracle):
    """TinyLlama dimensions (dim 2048, 32/4 heads, head_dim 64, ffn 5632, vocab 32000), 2 of its
    22 layers: 100 prompt positions through the MFMA GEMMs, then 3 greedy steps."""
    cfg = oracle.Config(dim=2048, n_layers=2, n_heads=32, n_kv_heads=4, ffn=5632, vocab=32000, ctx_len=256)
    w = oracle.synthetic_weights(cfg, 21)
    om = oracle.Model(cfg, w)
    prompt = oracle.prompt_tokens(100, cfg.vocab, 5)
    first, ologits, follow = oracle_prefill(om, prompt, 3)
    m = gpu_model(A, ctx, cfg, w)
    got = m.prefill(prompt)
    assert within_tol(m.logits(), ologits)
    assert got == first
    assert gpu_follow(m, prompt, got, 3) == follow
    m.close()


def test_prefill_library_gemms_tinyllama_width(A, ctx, oracle):
    """TinyLlama widths (dim 2048, 32/4 heads, ffn 5632; 2 layers, vocab 512) with a 264-position
    prompt: a chunk of 256 rows or more runs its F16 GEMMs on hipBLASLt (QKV stored straight, the
    gate/up pairs through the SwiGLU row kernel, O and down in f32 through the fused residual +
    RMSNorm rows). Next token, logits and the following greedy steps equal the per-position oracle."""
    cfg = oracle.Config(dim=2048, n_layers=2, n_heads=32, n_kv_heads=4, ffn=5632, vocab=512, ctx_len=300)
    w = oracle.synthetic_weights(cfg, 23)
    om = oracle.Model(cfg, w)
    prompt = oracle.prompt_tokens(264, cfg.vocab, 8)
    first, ologits, follow = oracle_prefill(om, prompt, 3)
    m = gpu_model(A, ctx, cfg, w)
    got = m.prefill(prompt)
    assert within_tol(m.logits(), ologits)
    assert got == first
    assert gpu_follow(m, prompt, got, 3) == follow
    m.close()


def test_prefill_long_chunk_llama3_width_matches_per_position(A, ctx, oracle):
    """Llama-3-8B widths (dim 4096, 32/8 heads, head_dim 128, ffn 14336; 1 layer, vocab 4096) with a
    300-row chunk (library GEMMs, matrix-core attention with 4 query heads per KV head): next token
    and logits equal the per-position forward_pass of the same weights (the decode kernels, which
    the other tests pin to the oracle)."""
    cfg = oracle.Config(dim=4096, n_layers=1, n_heads=32, n_kv_heads=8, ffn=14336, vocab=4096, ctx_len=320,
                        theta=500000.0)
    w = oracle.synthetic_weights(cfg, 19)
    prompt = oracle.prompt_tokens(300, cfg.vocab, 9)
    m = gpu_model(A, ctx, cfg, w)
    got = m.prefill(prompt)
    lp = m.logits().astype(np.float32)
    m.close()
    m = gpu_model(A, ctx, cfg, w)
    for p in range(len(prompt)):
        want = m.forward_pass(prompt, p)
    assert within_tol(lp, m.logits())
    assert got == want
    m.close()


def test_prefill_48_column_tiles(A, ctx, oracle):
    """dim 4096 (32 / 8 heads, head_dim 128) with ffn 1024: the QKV GEMM (6144 columns, 2 K splits
    into the fused QKV tail) and the down GEMM (residual epilogue, 2 K splits into the fused norm
    tail) take 48-column tiles, which fill more of the chip than 64-column ones; 100 prompt
    positions and 3 greedy steps against the per-position oracle."""
    cfg = oracle.Config(dim=4096, n_layers=1, n_heads=32, n_kv_heads=8, ffn=1024, vocab=512, ctx_len=128)
    w = oracle.synthetic_weights(cfg, 31)
    om = oracle.Model(cfg, w)
    prompt = oracle.prompt_tokens(100, cfg.vocab, 6)
    first, ologits, follow = oracle_prefill(om, prompt, 3)
    m = gpu_model(A, ctx, cfg, w)
    got = m.prefill(prompt)
    assert within_tol(m.logits(), ologits)
    assert got == first
    assert gpu_follow(m, prompt, got, 3) == follow
    m.close()


@pytest.mark.parametrize("dim,heads,kv,n_prompt,split", [(512, 8, 1, 150, 0), (512, 4, 1, 150, 0),
                                                        (1024, 8, 1, 140, 70),
                                                        # matrix-core attention (chunks of 256 rows
                                                        # or more): head_dim 64 / 128 with 8, 4, 2
                                                        # and 1 query heads per KV head, partial row
                                                        # blocks, continuations at start_pos > 0
                                                        (512, 8, 1, 300, 0), (256, 4, 1, 300, 0),
                                                        (256, 4, 2, 290, 0), (256, 4, 4, 400, 100),
                                                        (1024, 8, 1, 270, 0), (1024, 8, 2, 300, 0),
                                                        (512, 4, 2, 300, 0), (512, 4, 4, 280, 0),
                                                        (512, 8, 1, 420, 120)])
def test_prefill_grouped_attention_tiles(A, ctx, oracle, dim, heads, kv, n_prompt, split):
    """The GQA-grouped prefill attention: chunks under 256 rows on the tile kernel (one workgroup
    per row and KV head, 128-position LDS tiles; head_dim 64 with 8 query heads per KV head,
    head_dim 128 with 4 and with 8, a continuation at start_pos 70), longer chunks on the
    matrix-core kernel (every head_dim / group instance, row counts that leave the last row block
    partial, and second chunks of 300 rows after 100 or 120 positions). Next token, logits and
    the following greedy steps equal the per-position oracle."""
    cfg = oracle.Config(dim=dim, n_layers=2, n_heads=heads, n_kv_heads=kv, ffn=2 * dim, vocab=512,
                        ctx_len=n_prompt + 16)
    w = oracle.synthetic_weights(cfg, 77)
    om = oracle.Model(cfg, w)
    prompt = oracle.prompt_tokens(n_prompt, cfg.vocab, 3)
    first, ologits, follow = oracle_prefill(om, prompt, 3)
    m = gpu_model(A, ctx, cfg, w)
    if split:
        m.prefill(prompt[:split])
        got = m.prefill(prompt[split:], start_pos=split)
    else:
        got = m.prefill(prompt)
    assert within_tol(m.logits(), ologits)
    assert got == first
    assert gpu_follow(m, prompt, got, 3) == follow
    m.close()


def test_generate_with_batched_prefill_matches_golden(A, ctx, oracle):
    """The committed tiny-model stream (16-token prompt, 64 greedy tokens) with batched prefill."""
    import os

    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "tiny_stream.npz"))
    cfg = oracle.TINY
    m = gpu_model(A, ctx, cfg, oracle.synthetic_weights(cfg, int(g["seed"])))
    toks, reason = m.generate(g["prompt"].tolist(), int(g["n_new"]), batched_prefill=True)
    assert toks == g["tokens"].tolist() and reason == "length"
    m.close()


def test_prefill_errors(A, ctx, oracle):
    cfg = oracle.TINY
    m = A.Model.create(ctx, A.ModelConfig(cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.ffn, cfg.vocab,
                                          cfg.ctx_len))
    with pytest.raises(A.AesirError, match="outside the embedding vocabulary"):
        m.prefill([1, cfg.vocab])
    with pytest.raises(A.AesirError, match="exceeds the model context length"):
        m.prefill([1] * 10, start_pos=cfg.ctx_len - 5)
    assert m.prefill([]) == 0
    m.close()
