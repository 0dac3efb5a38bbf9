"""GPU parity of the GGUF block formats beyond Q4_0 / Q4_K / Q6_K / Q8_0: Q4_1, Q5_0, Q5_1 (the
reference's BlockQ4_1 / BlockQ5_0 / BlockQ5_1 with its gemm_q4_1 / _q5_0 / _q5_1 arithmetic,
core/compute.mojo:914-1036) and GGML's Q2_K, Q3_K and Q5_K super-blocks, all repacked like Q4_0 /
Q4_K (their GEMV, prefill and model paths are in the Q4_0 / Q4_K tests' parametrization): the
error texts of aesir_gemm_quant, and a model of each type whose every matrix reads back as the
oracle's f16 weights, bit for bit.
"""
import numpy as np
import pytest

from quant_tools import expected_f16, make_tensor, same_token

pytestmark = pytest.mark.gpu

NEW = {"q4_1": 3, "q5_0": 6, "q5_1": 7, "q2_k": 10, "q3_k": 11, "q5_k": 13}


@pytest.fixture(scope="module")
def A():
    import aesir_hip

    return aesir_hip


@pytest.fixture(scope="module")
def ctx(A):
    c = A.Context(2 << 30)
    yield c
    c.close()


@pytest.fixture(autouse=True)
def well_scope(ctx):
    off = ctx.offset
    yield
    ctx.synchronize()
    ctx.reset(off)


def test_gemm_quant_formats_errors(A, ctx):
    a = ctx.tensor(1, 96)
    c = ctx.tensor(1, 2)
    with pytest.raises(A.AesirError, match="gemm_q5_1: inner dimension must be a multiple of 32"):
        A.gemm_quant(ctx, ctx.tensor(1, 40), a.ptr, 7, 2, c)
    with pytest.raises(A.AesirError, match="gemm_q3_k: inner dimension must be a multiple of 256"):
        A.gemm_quant(ctx, a, a.ptr, 11, 2, c)
    with pytest.raises(A.AesirError, match="gemm_q4_1: output matrix shape mismatch"):
        A.gemm_quant(ctx, ctx.tensor(1, 64), a.ptr, 3, 3, c)


@pytest.mark.parametrize("kind", list(NEW))
def test_model_of_each_format(A, ctx, oracle, kind):
    """A model whose matrices all have the type: every matrix reads back as the oracle's f16
    weights bit for bit; weight_type names the type; the greedy tokens follow the oracle on those
    weights and graph replay equals eager launches."""
    cfg = oracle.Config(dim=256, n_layers=1, n_heads=4, n_kv_heads=2, ffn=512, vocab=64, ctx_len=32)
    m = A.Model.create(ctx, A.ModelConfig(cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.ffn, cfg.vocab,
                                          cfg.ctx_len), NEW[kind])
    assert m.weight_type == NEW[kind]
    rng = np.random.default_rng(NEW[kind])
    w = {}
    for name, (r, c) in oracle.tensor_shapes(cfg).items():
        if name.endswith("norm.weight"):
            w[name] = (1.0 + 0.05 * rng.standard_normal(c)).astype(np.float16)
        else:
            w[name] = make_tensor(A, NEW[kind], r, c, rng)
            assert m.tensor_type(name) == NEW[kind]
    m.set_weights(w)
    back = {}
    for name, shape in oracle.tensor_shapes(cfg).items():
        back[name] = m.get_tensor(name, shape)
        if not name.endswith("norm.weight"):
            want = expected_f16(oracle, NEW[kind], w[name])
            assert np.array_equal(back[name].view(np.uint16), want.view(np.uint16)), (kind, name)
    om = oracle.Model(cfg, back)
    okv = om.new_kv()
    cur = [3, 9, 27]
    for p in range(3):
        want, ol = om.forward(okv, cur, p)
        assert same_token(m.forward_pass(cur, p), want, ol), (kind, p)
    g, _ = m.decode_loop(5, 3, 8, use_graph=True)
    e, _ = m.decode_loop(5, 3, 8, use_graph=False)
    assert g == e
    m.close()
