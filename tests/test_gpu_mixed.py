"""GPU parity of models whose matrices differ in type (aesir_model_create_mixed, and GGUF files that
mix types, as Q4_K_M files do) against the CPU oracle.

- Every matrix read back (get_tensor) equals, bit for bit, the oracle's f16 dequantization of the
  blocks uploaded for it: its own type's rule where the matrix keeps its type, and each part's
  rule where a fused matrix (Q/K/V, gate/up) of differing parts is stored in f16.
- The model then computes what the F16 oracle holding those weights computes: per-position
  forward passes (logits within the forward-pass tolerance, tokens equal but at near ties of the
  oracle's logits), graph replay == eager launches == the host loop, batched prefill against
  per-position.
- A GGUF file holding the same tensors loads into the same model.
"""
import numpy as np
import pytest

from quant_tools import (F16, Q2_K, Q3_K, Q4_0, Q4_1, Q4_K, Q5_0, Q5_1, Q5_K, Q6_K, Q8_0, expected_f16, make_tensor,
                         same_token, within_tol)

pytestmark = pytest.mark.gpu

PER = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")


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


def layout(embd, out, layers):
    t = {"token_embd.weight": embd, "output.weight": out}
    for l, types in enumerate(layers):
        for b, v in zip(PER, types):
            t[f"blk.{l}.{b}.weight"] = v
    return t


# (q, k, v, o, gate, up, down) per layer
MIXES = {
    # embedding table of another type than layer 0's Q/K/V (stored f16: V differs): looked up first
    "embd_apart": layout(Q4_K, Q6_K, [(Q4_K, Q4_K, Q6_K, Q4_K, Q4_K, Q4_K, Q6_K),
                                      (Q4_K, Q4_K, Q4_K, Q8_0, Q4_0, Q4_K, F16)]),
    # embedding fused into layer 0's Q/K/V GEMV (both Q6_K); f16 Q/K/V from F16 and Q8_0 parts
    "embd_fused": layout(Q6_K, Q8_0, [(Q6_K, Q6_K, Q6_K, F16, Q8_0, Q8_0, Q4_0),
                                      (F16, F16, Q8_0, Q6_K, F16, F16, Q4_K)]),
    # F16 embedding and Q/K/V in a model with quantized matrices elsewhere
    "f16_front": layout(F16, Q4_0, [(F16, F16, F16, Q6_K, Q4_K, Q4_K, Q8_0),
                                    (Q8_0, Q8_0, Q8_0, Q4_0, Q6_K, Q6_K, Q4_K)]),
    # the other GGUF formats: Q4_1, Q5_0, Q5_1, Q5_K, Q2_K and Q3_K repacked as standalone matrices
    # (Q5_0 Q/K/V fused, the Q5_K table looked up apart, a Q2_K down, a Q3_K O and lm_head), and
    # layer 1's Q5_K / Q6_K Q/K/V in two parts (Q and K in Q5_K, V in Q6_K)
    "more_types": layout(Q5_K, Q3_K, [(Q5_0, Q5_0, Q5_0, Q4_1, Q5_1, Q5_1, Q2_K),
                                      (Q5_K, Q5_K, Q6_K, Q3_K, Q4_K, Q4_K, Q5_0)]),
    # fused matrices whose parts are Q2_K and Q3_K: Q/K/V and gate/up stored in f16, each part
    # dequantized by its own type's rule
    "kquant_parts_f16": layout(Q4_K, Q2_K, [(Q3_K, Q2_K, Q3_K, Q2_K, Q2_K, Q3_K, Q3_K),
                                            (Q2_K, Q3_K, Q2_K, Q3_K, Q3_K, Q2_K, Q2_K)]),
    # Q/K/V in two parts read by one two-part launch: Q alone, K and V in another type (Q2_K | Q4_K),
    # and Q and K in one type, V in another (Q3_K | Q5_K)
    "qkv_two_parts_a": layout(Q4_K, Q6_K, [(Q2_K, Q4_K, Q4_K, Q4_K, Q4_K, Q4_K, Q6_K),
                                           (Q3_K, Q3_K, Q5_K, Q4_K, Q5_K, Q5_K, Q4_K)]),
    # the other pairs: Q4_K | Q5_K and Q3_K | Q4_K
    "qkv_two_parts_b": layout(Q5_K, Q4_K, [(Q4_K, Q4_K, Q5_K, Q6_K, Q4_K, Q4_K, Q5_K),
                                           (Q3_K, Q4_K, Q4_K, Q4_K, Q6_K, Q6_K, Q4_K)]),
}

SMALL = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, ffn=512, vocab=300, ctx_len=160)


def mixed_weights(A, oracle, cfg, types, rng):
    w = {}
    for name, (r, c) in oracle.tensor_shapes(cfg).items():
        if name.endswith("norm.weight"):
            w[name] = (1.0 + 0.05 * rng.standard_normal(c)).astype(np.float16)
        else:
            w[name] = make_tensor(A, types[name], r, c, rng)
    return w


def model_cfg(A, cfg):
    return A.ModelConfig(cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.ffn, cfg.vocab, cfg.ctx_len,
                         cfg.eps, cfg.theta, 1, -1)


def mixed_model(A, ctx, oracle, cfg, types, seed):
    rng = np.random.default_rng(seed)
    w = mixed_weights(A, oracle, cfg, types, rng)
    m = A.Model.create_mixed(ctx, model_cfg(A, cfg), types)
    m.set_weights(w)
    back = {name: m.get_tensor(name, shape) for name, shape in oracle.tensor_shapes(cfg).items()}
    return m, w, back


@pytest.mark.parametrize("mix", list(MIXES))
def test_mixed_read_back_is_each_types_rule(A, ctx, oracle, mix):
    cfg = oracle.Config(**SMALL)
    types = MIXES[mix]
    m, w, back = mixed_model(A, ctx, oracle, cfg, types, 3)
    assert m.weight_type == A.WEIGHT_MIXED
    for name, x in w.items():
        if name.endswith("norm.weight"):
            assert np.array_equal(back[name].reshape(-1).view(np.uint16), x.view(np.uint16)), name
            assert m.tensor_type(name) == F16
            continue
        assert m.tensor_type(name) == types[name], name
        want = expected_f16(oracle, types[name], x)
        assert np.array_equal(back[name].view(np.uint16), want.view(np.uint16)), (mix, name)
    m.close()


@pytest.mark.parametrize("mix", list(MIXES))
def test_mixed_model_stream_matches_oracle(A, ctx, oracle, mix):
    """Per-position forward passes, then graph-replayed decode, against the F16 oracle on the
    read-back weights; graph replay == eager launches == the host loop."""
    cfg = oracle.Config(**SMALL)
    m, _, back = mixed_model(A, ctx, oracle, cfg, MIXES[mix], 5)
    om = oracle.Model(cfg, back)
    prompt = oracle.prompt_tokens(12, cfg.vocab, 3)
    okv = om.new_kv()
    cur = list(prompt)
    for p in range(len(prompt) + 16):
        want, ol = om.forward(okv, cur, p)
        got = m.forward_pass(cur, p)
        assert within_tol(m.logits(), ol), (mix, p)
        assert same_token(got, want, ol), (mix, p, got, want)
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


@pytest.mark.parametrize("mix", list(MIXES))
def test_mixed_batched_prefill_matches_per_position(A, ctx, oracle, mix):
    """aesir_prefill of a 140-token prompt (one chunk: two 128-row M tiles of the wide GEMM) against
    the per-position oracle."""
    cfg = oracle.Config(**SMALL)
    m, _, back = mixed_model(A, ctx, oracle, cfg, MIXES[mix], 6)
    om = oracle.Model(cfg, back)
    prompt = oracle.prompt_tokens(140, cfg.vocab, 4)
    okv = om.new_kv()
    for p in range(len(prompt)):
        want, ol = om.forward(okv, prompt, p)
    got = m.prefill(prompt, 0)
    assert within_tol(m.logits(), ol)
    assert same_token(got, want, ol), (got, want)
    m.close()


@pytest.mark.parametrize("mix", list(MIXES))
def test_mixed_long_chunk_prefill_matches_per_position(A, ctx, oracle, mix):
    """A 300-row chunk of every mix: each matrix (a two-part Q/K/V as one f16 copy of both parts)
    dequantized and multiplied on hipBLASLt, against the per-position oracle."""
    cfg = oracle.Config(**{**SMALL, "ctx_len": 320})
    m, _, back = mixed_model(A, ctx, oracle, cfg, MIXES[mix], 8)
    om = oracle.Model(cfg, back)
    prompt = oracle.prompt_tokens(300, cfg.vocab, 6)
    okv = om.new_kv()
    for p in range(len(prompt)):
        want, ol = om.forward(okv, prompt, p)
    got = m.prefill(prompt, 0)
    assert within_tol(m.logits(), ol)
    assert same_token(got, want, ol), (got, want)
    m.close()


@pytest.mark.parametrize("mix", ["embd_apart", "more_types"])
def test_mixed_gguf_file_loads_like_set_tensor(A, ctx, oracle, tmp_path, mix):
    from gguf_tools import llama_metadata, write_gguf

    cfg = oracle.Config(**SMALL)
    types = MIXES[mix]
    rng = np.random.default_rng(7)
    w = mixed_weights(A, oracle, cfg, types, rng)
    tensors = {k: (v.astype(np.float32) if k.endswith("norm.weight") else v) for k, v in w.items()}
    path = str(tmp_path / "mixed.gguf")
    write_gguf(path, llama_metadata(cfg, cfg.vocab), tensors)
    mf = A.Model.load_gguf(ctx, path, cfg.ctx_len)
    assert mf.weight_type == A.WEIGHT_MIXED
    ms = A.Model.create_mixed(ctx, A.ModelConfig(cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.ffn,
                                                 cfg.vocab, cfg.ctx_len, cfg.eps, cfg.theta, 1, 2), types)
    ms.set_weights(w)
    for name, shape in oracle.tensor_shapes(cfg).items():
        assert mf.tensor_type(name) == ms.tensor_type(name), name
        assert np.array_equal(mf.get_tensor(name, shape), ms.get_tensor(name, shape)), name
    prompt = oracle.prompt_tokens(6, cfg.vocab, 8)
    a, _ = mf.generate(prompt, 8)
    b, _ = ms.generate(prompt, 8)
    assert a == b
    mf.close()
    ms.close()


def test_mixed_errors(A, ctx, oracle):
    cfg = oracle.Config(**SMALL)
    with pytest.raises(ValueError, match="not a model matrix"):
        A.Model.create_mixed(ctx, model_cfg(A, cfg), {"blk.9.attn_q.weight": Q4_K})
    bad = A.ModelConfig(160, 1, 4, 4, 256, 64, 16)  # Q4_K needs dim % 256 == 0
    with pytest.raises(A.AesirError, match="Q4_K weights need dim and ffn to be multiples of 256"):
        A.Model.create_mixed(ctx, bad, {"blk.0.ffn_down.weight": Q4_K})
    with pytest.raises(A.AesirError, match="weight type 15 is not F16, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1"):
        A.Model.create_mixed(ctx, model_cfg(A, cfg), {"output.weight": 15})  # GGML Q8_K
    m = A.Model.create_mixed(ctx, model_cfg(A, cfg), MIXES["embd_apart"])
    with pytest.raises(A.AesirError, match="invalid type: blk.0.attn_v.weight"):
        m.set_tensor("blk.0.attn_v.weight", np.zeros((cfg.kv_dim, cfg.dim), np.float16))
    with pytest.raises(A.AesirError, match="invalid type: blk.1.ffn_down.weight"):
        m.set_tensor("blk.1.ffn_down.weight", make_tensor(A, Q8_0, cfg.dim, cfg.ffn, np.random.default_rng(0)))
    m.close()


def q4_k_m_types(n_layers):
    """llama.cpp's Q4_K_M recipe: Q4_K everywhere, Q6_K for output and for attn_v / ffn_down of the
    first and last eighth of the layers and every third layer between."""
    more = lambda l: l < n_layers // 8 or l >= 7 * n_layers // 8 or (l - n_layers // 8) % 3 == 2
    layers = [(Q4_K, Q4_K, Q6_K if more(l) else Q4_K, Q4_K, Q4_K, Q4_K, Q6_K if more(l) else Q4_K)
              for l in range(n_layers)]
    return layout(Q4_K, Q6_K, layers)


@pytest.mark.timeout(600)
def test_q4_k_m_llama3_8b_shape_properties(A, oracle):
    """Llama-3-8B shape in the Q4_K_M layout with device-initialized weights: graph == eager ==
    forward_pass for 6 steps from KV 2048, finite logits, matrices read back within their range."""
    cfg = oracle.LLAMA3_8B
    with A.Context(16 << 30) as big:
        m = A.Model.create_mixed(big, A.ModelConfig(cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.ffn,
                                                    cfg.vocab, 2048 + 16), q4_k_m_types(cfg.n_layers))
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
        for name in ("blk.0.attn_q.weight", "blk.0.ffn_down.weight", "blk.5.ffn_down.weight"):
            r, c = (cfg.dim, cfg.ffn) if "down" in name else (cfg.dim, cfg.dim)
            wd = m.get_tensor(name, (r, c)).astype(np.float32)
            assert np.isfinite(wd).all() and 0.01 < wd.std() < 0.04, (name, wd.std())
        m.close()
