"""GPU parity of the Q8_0 weight path (GGUF type-8 matrices decoded on the device).

A Q8_0 model uses every weight as w = f16(f16(q) * d), gemm_q8_0's rule
(core/compute.mojo:1038-1065), so it must compute what the F16 oracle computes with the
dequantized weights: identical greedy tokens, logits within max-abs 2e-2 / rel 1e-2. Covered:
- the read-back of every matrix equals the host dequantization bit for bit (repacking into
  quants + scales loses nothing; fused Q|K|V and interleaved gate/up placement included);
- shapes where K < 4096 (idle threads), K = 4096, partial last slabs (K = 5632, 14336, 16896)
  and the longest row, K = 28672; the Q8_0 embedding row fused into layer 0, and the Q8_0
  lm_head with its argmax;
- a GGUF v3 file with Q8_0 matrices loads into the same model as set_tensor builds;
- graph replay equals eager launches; the batched prefill (Q8_0 MFMA GEMMs) equals the
  per-position oracle; device init draws quants and scales in their stated ranges.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q8_SMALL = dict(dim=128, n_layers=2, n_heads=4, n_kv_heads=2, ffn=256, vocab=500, ctx_len=128)
Q8_TL = dict(dim=2048, n_layers=2, n_heads=32, n_kv_heads=4, ffn=5632, vocab=32000, ctx_len=64)
Q8_L3 = dict(dim=4096, n_layers=1, n_heads=32, n_kv_heads=8, ffn=14336, vocab=4096, ctx_len=32)
# rows past 16384 weights: five 4096-wide slabs (the last partial) in QKV, O and the lm_head; seven
# in ffn_down at a 70B-class ffn of 28672, the longest row the Q8_0 decode GEMV takes
Q8_WIDE = dict(dim=16896, n_layers=1, n_heads=132, n_kv_heads=11, ffn=256, vocab=256, ctx_len=16)
Q8_LONG_FFN = dict(dim=256, n_layers=1, n_heads=4, n_kv_heads=2, ffn=28672, vocab=256, ctx_len=16)


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


def q8_weights(A, oracle, cfg, seed):
    """Q8_0 matrices (q uniform in [-127, 127], d uniform in [0.5, 1.5) * 0.02 / 64, so weights
    of standard deviation near 0.02) and f16 norms. Returns (GPU tensors, dequantized f16 dict)."""
    rng = np.random.default_rng(seed)
    norms = oracle.synthetic_weights(oracle.Config(**cfg), seed)
    gpu, deq = {}, {}
    for name, (r, c) in oracle.tensor_shapes(oracle.Config(**cfg)).items():
        if name.endswith("norm.weight"):
            gpu[name] = deq[name] = norms[name]
            continue
        q = rng.integers(-127, 128, size=(r, c), dtype=np.int8)
        d = ((0.5 + rng.random((r, c // 32))) * (0.02 / 64)).astype(np.float16)
        t = A.Q8_0Tensor.from_parts(d, q)
        gpu[name] = t
        deq[name] = t.dequantize()
    return gpu, deq


def q8_model(A, ctx, cfg, tensors):
    mc = A.ModelConfig(cfg["dim"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"], cfg["ffn"], cfg["vocab"],
                       cfg["ctx_len"], 1e-5, 10000.0, 1, -1)
    m = A.Model.create(ctx, mc, A.GGML_Q8_0)
    m.set_weights(tensors)
    return m


def oracle_stream(om, prompt, n_new):
    kv = om.new_kv()
    cur = list(prompt)
    logits = []
    nxt = None
    for p in range(len(prompt)):
        nxt, lg = om.forward(kv, cur, p)
    logits.append(lg)
    out = []
    for _ in range(n_new):
        out.append(nxt)
        cur.append(nxt)
        if len(out) == n_new:
            break
        nxt, lg = om.forward(kv, cur, len(cur) - 1)
        logits.append(lg)
    return out, logits


def gpu_stream(m, prompt, n_new):
    cur = list(prompt)
    nxt = None
    for p in range(len(prompt)):
        nxt = m.forward_pass(cur, p)
    logits = [m.logits()]
    out = []
    for _ in range(n_new):
        out.append(nxt)
        cur.append(nxt)
        if len(out) == n_new:
            break
        nxt = m.forward_pass(cur, len(cur) - 1)
        logits.append(m.logits())
    return out, logits


def test_q8_small_model_matches_dequantized_oracle(A, ctx, oracle):
    cfg = Q8_SMALL
    tensors, deq = q8_weights(A, oracle, cfg, 11)
    m = q8_model(A, ctx, cfg, tensors)
    assert m.weight_type == A.GGML_Q8_0
    for name, w in deq.items():
        got = m.get_tensor(name, w.shape)
        assert np.array_equal(got.view(np.uint16), np.asarray(w, np.float16).view(np.uint16)), name
    om = oracle.Model(oracle.Config(**cfg), deq)
    prompt = oracle.prompt_tokens(16, cfg["vocab"], 3)
    want, wl = oracle_stream(om, prompt, 24)
    got, gl = gpu_stream(m, prompt, 24)
    assert got == want
    for a, b in zip(gl, wl):
        assert within_tol(a, b)
    m.close()


@pytest.mark.parametrize("shape", ["tinyllama", "llama3", "wide", "long_ffn"])
def test_q8_model_shapes_match_dequantized_oracle(A, ctx, oracle, shape):
    """K = 2048 (half the threads idle) and 5632 (partial second slab); K = 4096 and 14336
    (partial fourth slab); K = 16896 (partial fifth slab) and 28672 (seven slabs)."""
    cfg = {"tinyllama": Q8_TL, "llama3": Q8_L3, "wide": Q8_WIDE, "long_ffn": Q8_LONG_FFN}[shape]
    tensors, deq = q8_weights(A, oracle, cfg, 5)
    m = q8_model(A, ctx, cfg, tensors)
    om = oracle.Model(oracle.Config(**cfg), deq)
    prompt = oracle.prompt_tokens(4, cfg["vocab"], 9)
    want, wl = oracle_stream(om, prompt, 3)
    got, gl = gpu_stream(m, prompt, 3)
    assert got == want
    for a, b in zip(gl, wl):
        assert within_tol(a, b)
    m.close()


def test_q8_gguf_load_matches_set_tensor(A, ctx, oracle, tmp_path):
    from gguf_tools import T_FLOAT32, llama_metadata, write_gguf

    cfg = Q8_SMALL
    tensors, deq = q8_weights(A, oracle, cfg, 23)
    oc = oracle.Config(**cfg)
    file_tensors = {k: (v.reshape(-1).astype(np.float32) if k.endswith("norm.weight") else v)
                    for k, v in tensors.items()}
    path = str(tmp_path / "q8.gguf")
    write_gguf(path, llama_metadata(oc, cfg["vocab"]), file_tensors)
    c, _ = A.gguf_inspect(path)
    assert (c.dim, c.ffn, c.vocab) == (cfg["dim"], cfg["ffn"], cfg["vocab"])
    g = A.Model.load_gguf(ctx, path, cfg["ctx_len"])
    assert g.weight_type == A.GGML_Q8_0
    m = q8_model(A, ctx, cfg, tensors)
    prompt = oracle.prompt_tokens(8, cfg["vocab"], 4)
    a, _ = gpu_stream(g, prompt, 12)
    b, _ = gpu_stream(m, prompt, 12)
    assert a == b
    w, _ = oracle_stream(oracle.Model(oc, deq), prompt, 12)
    assert a == w
    g.close()
    m.close()


def test_q8_graph_eager_prefill_agree(A, ctx, oracle):
    """Device-autoregressive decode (graph and eager) continues the host-driven stream; the
    batched prefill returns the same next token."""
    cfg = Q8_TL
    tensors, _ = q8_weights(A, oracle, cfg, 31)
    m = q8_model(A, ctx, cfg, tensors)
    prompt = oracle.prompt_tokens(6, cfg["vocab"], 2)
    host, _ = gpu_stream(m, prompt, 8)
    m2 = q8_model(A, ctx, cfg, tensors)
    assert m2.prefill(prompt) == host[0]
    pos = len(prompt)
    g_toks, _ = m2.decode_loop(host[0], pos, 7, use_graph=True)
    assert list(g_toks) == host[1:]
    m3 = q8_model(A, ctx, cfg, tensors)
    m3.prefill(prompt)
    e_toks, _ = m3.decode_loop(host[0], pos, 7, use_graph=False)
    assert list(e_toks) == host[1:]
    for mm in (m, m2, m3):
        mm.close()


@pytest.mark.parametrize("shape,n_prompt,split", [("small", 40, 0), ("small", 200, 77), ("tinyllama", 100, 0),
                                                   ("small", 300, 0), ("small", 420, 120)])
def test_q8_batched_prefill_matches_per_position(A, ctx, oracle, shape, n_prompt, split):
    """aesir_prefill on a Q8_0 model runs the Q8_0 MFMA GEMMs (quants and scales copied into LDS,
    dequantized per fragment): the next token, logits within tolerance and the greedy steps that
    read the prefilled cache equal the per-position oracle on the dequantized weights. 200
    positions = one chunk of two 128-row M tiles; `split` > 0 prefills the prompt in two calls
    (start_pos > 0). Chunks of 300 rows take the long-chunk path instead: the matrices
    dequantized to f16 (f16(f16(q) d)) and multiplied on hipBLASLt."""
    cfg = dict(Q8_SMALL if shape == "small" else Q8_TL)
    cfg["ctx_len"] = max(cfg["ctx_len"], n_prompt + 8)
    tensors, deq = q8_weights(A, oracle, cfg, 41)
    om = oracle.Model(oracle.Config(**cfg), deq)
    prompt = oracle.prompt_tokens(n_prompt, cfg["vocab"], 13)
    want, wl = oracle_stream(om, prompt, 3)
    m = q8_model(A, ctx, cfg, tensors)
    if split:
        m.prefill(prompt[:split])
        got = m.prefill(prompt[split:], start_pos=split)
    else:
        got = m.prefill(prompt)
    assert within_tol(m.logits(), wl[0])
    assert got == want[0]
    cur = list(prompt) + [got]
    follow = [got]
    for _ in range(2):
        nxt = m.forward_pass(cur, len(cur) - 1)
        cur.append(nxt)
        follow.append(nxt)
    assert follow == want
    m.close()


def test_q8_init_random_ranges(A, ctx):
    cfg = Q8_SMALL
    mc = A.ModelConfig(cfg["dim"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"], cfg["ffn"], cfg["vocab"],
                       cfg["ctx_len"])
    m = A.Model.create(ctx, mc, A.GGML_Q8_0)
    m.init_random(7, std=0.02)
    w = m.get_tensor("blk.1.ffn_down.weight", (cfg["dim"], cfg["ffn"])).astype(np.float64)
    bound = 127 * 1.5 * 0.02 / 64 * (1 + 2.0 ** -10)
    assert np.all(np.abs(w) <= bound)
    assert 0.015 < w.std() < 0.03
    assert len(np.unique(w)) > 1000
    assert m.forward_pass([1, 2, 3], 2) >= 0
    assert np.all(np.isfinite(m.logits().astype(np.float32)))
    t = m.kernel_times(5, 3)
    assert all(v > 0 for v in t.values())
    m.close()


def test_q8_errors(A, ctx):
    bad = A.ModelConfig(80, 1, 4, 4, 256, 64, 16)
    with pytest.raises(A.AesirError, match="Q8_0 weights need dim and ffn to be multiples of 32"):
        A.Model.create(ctx, bad, A.GGML_Q8_0)
    with pytest.raises(A.AesirError, match="weight type 9 is not F16, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q2_K"):
        A.Model.create(ctx, A.ModelConfig(64, 1, 4, 4, 64, 64, 16), 9)  # GGML Q8_1
    m = A.Model.create(ctx, A.ModelConfig(64, 1, 4, 4, 64, 64, 16), A.GGML_Q8_0)
    with pytest.raises(A.AesirError, match="invalid type: blk.0.attn_q.weight"):
        m.set_tensor("blk.0.attn_q.weight", np.zeros((64, 64), np.float16))
    m.set_tensor("blk.0.attn_norm.weight", np.ones(64, np.float32))  # norms stay F32/F16
    m.close()
