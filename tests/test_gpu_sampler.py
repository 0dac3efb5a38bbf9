"""GPU parity of the sampler stack (aesir_sample_token, sample_token_from_logits at
core/sampler.mojo:217-305) against the CPU oracle: the sampled token and the RuneRNG state must be
identical, draw after draw, for every stage combination (greedy branch, penalties, temperature,
top-k, top-p, min-p, suppress list), at vocabulary sizes from 512 to 300000 (1000 and 4099 end in
a short 32-term block and a short chunk of the draw, 4099 also in a short LDS tile of the
truncations), with many tied logits so the stable-sort order is exercised. Both sides compute exp
as the correctly rounded f32 value and keep the reference's sequential f32 sums, so equality is
exact. The device evaluates the final draw's running sum in parallel (one integer add per chunk
wherever no rounding depends on the order); these tests are what pin that to the sequential
sum."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def A():
    import aesir_hip

    return aesir_hip


@pytest.fixture(scope="module")
def ctx(A):
    c = A.Context(256 << 20)
    yield c
    c.close()


@pytest.fixture(autouse=True)
def well_scope(ctx):
    off = ctx.offset
    yield
    ctx.synchronize()
    ctx.reset(off)


CONFIGS = [
    dict(temperature=0.0),
    dict(temperature=0.8, top_k=1),
    dict(temperature=1.0),
    dict(temperature=0.7),
    dict(temperature=1.2, top_k=40),
    dict(temperature=0.9, top_p=0.9),
    dict(temperature=1.0, top_k=50, top_p=0.95, min_p=0.05),
    dict(temperature=1.5, min_p=0.1),
    dict(temperature=0.8, top_k=200, repetition_penalty=1.3, frequency_penalty=0.2, presence_penalty=0.4),
    dict(temperature=1.1, top_p=0.5, repetition_penalty=0.8),
    # more candidates than one LDS tile after top-k: the truncations and the draw run as chunked
    # stages (exact parallel running sums, device-side candidate counts)
    dict(temperature=1.0, top_k=5000),
    dict(temperature=0.9, top_k=5000, top_p=0.9),
    dict(temperature=1.2, top_k=6000, min_p=0.02),
    dict(temperature=0.8, top_p=0.95, min_p=0.01, frequency_penalty=0.3),
    # 1 / temperature overflows to inf: zero logits become NaN, sum_e is NaN, and the reference
    # still consumes the random number and returns its last candidate
    dict(temperature=1e-39),
]


@pytest.mark.parametrize("vocab", [512, 1000, 4099, 32000, 128256])
@pytest.mark.parametrize("cfgd", CONFIGS)
def test_sampler_matches_oracle(A, ctx, oracle, vocab, cfgd):
    rng = np.random.default_rng(vocab + len(cfgd))
    gcfg, ocfg = A.SamplerConfig(**cfgd), oracle.SamplerConfig(**cfgd)
    g_rng = A.RuneRNG(1234)
    o_state = oracle.rune_rng_state(1234)
    draws = 12 if vocab > 100000 else 24
    for d in range(draws):
        # logits on a coarse grid (ties) plus a few outliers; some non-finite values
        logits = (rng.integers(-40, 40, vocab) * 0.25).astype(np.float16)
        logits[rng.integers(0, vocab, 3)] = np.float16(12.0)
        logits[rng.integers(0, vocab, 2)] = np.inf
        logits[rng.integers(0, vocab, 2)] = np.nan
        context = rng.integers(0, vocab, 64).tolist()
        suppress = rng.integers(0, vocab, 4).tolist() + [vocab + 5]
        t = ctx.from_numpy(logits.reshape(1, -1))
        got = A.sample_token(ctx, t, gcfg, g_rng, context, suppress)
        want, o_state = oracle.sample_token_f16(logits, ocfg, o_state, context, suppress)
        assert got == want, (d, got, want)
        assert g_rng.state == o_state, d


def test_sampler_known_answers(A, ctx):
    """tests/test_inference.mojo:168-223 through the whole stack: top-k keeps ids 1 and 2 of
    [1, 5, 3]; top-p 0.9 keeps only id 0 of [10, 0, -10]; min-p 0.1 keeps only id 0 of [10, 2, -5]."""
    rng = A.RuneRNG(3)
    for _ in range(20):
        t = ctx.from_numpy(np.array([[1.0, 5.0, 3.0]], np.float16))
        assert A.sample_token(ctx, t, A.SamplerConfig(top_k=2), rng) in (1, 2)
        t = ctx.from_numpy(np.array([[10.0, 0.0, -10.0]], np.float16))
        assert A.sample_token(ctx, t, A.SamplerConfig(top_p=0.9), rng) == 0
        t = ctx.from_numpy(np.array([[10.0, 2.0, -5.0]], np.float16))
        assert A.sample_token(ctx, t, A.SamplerConfig(min_p=0.1), rng) == 0


def test_sampler_greedy_consumes_no_random_number(A, ctx, oracle):
    x = np.array([[1.0, np.inf, 2.0, np.nan, 2.0]], np.float16)
    rng = A.RuneRNG(5)
    st = rng.state
    assert A.sample_token(ctx, ctx.from_numpy(x), A.SamplerConfig(temperature=0.0), rng, suppress_tokens=[2]) == 4
    assert rng.state == st
    A.sample_token(ctx, ctx.from_numpy(x), A.SamplerConfig(temperature=1.0), rng)
    assert rng.state != st


@pytest.mark.parametrize("cfgd", [dict(temperature=1.0), dict(temperature=0.7, top_k=20000),
                                  dict(temperature=1.3, repetition_penalty=1.2), dict(temperature=0.9, top_p=0.9),
                                  dict(temperature=1.0, min_p=0.05)])
def test_sampler_long_vocabulary_matches_oracle(A, ctx, oracle, cfgd):
    """300000 candidates: the final draw's walk over chunk headers takes three rounds of LDS
    staging (131072 candidates each) and stores its recorded running sums in several groups of
    64; logits in N(0, 2) rounded to f16, as a model's are."""
    vocab = 300000
    rng = np.random.default_rng(77)
    gcfg, ocfg = A.SamplerConfig(**cfgd), oracle.SamplerConfig(**cfgd)
    g_rng = A.RuneRNG(99)
    o_state = oracle.rune_rng_state(99)
    for d in range(4):
        logits = (rng.standard_normal(vocab) * 2.0).astype(np.float16)
        context = rng.integers(0, vocab, 128).tolist()
        t = ctx.from_numpy(logits.reshape(1, -1))
        got = A.sample_token(ctx, t, gcfg, g_rng, context)
        want, o_state = oracle.sample_token_f16(logits, ocfg, o_state, context, [])
        assert got == want, (d, got, want)
        assert g_rng.state == o_state, d


@pytest.mark.parametrize("vocab", [4097, 10000, 128256])
@pytest.mark.parametrize("top_k", [2, 3, 4095, 4096])
@pytest.mark.parametrize("logit_kind", ["equal", "two_values", "grid"])
def test_sampler_topk_selection_matches_oracle(A, ctx, oracle, vocab, top_k, logit_kind):
    """top_k <= 4096 takes the first top_k of the stable descending sort without sorting the
    vocabulary (radix select of the k-th key, index-order compaction, a sort of the k selected).
    Ties at the threshold key must keep the lowest indices: all-equal logits (every key equals the
    threshold), two values, and a coarse grid."""
    rng = np.random.default_rng(vocab + top_k)
    cfgd = dict(temperature=0.9, top_k=top_k)
    gcfg, ocfg = A.SamplerConfig(**cfgd), oracle.SamplerConfig(**cfgd)
    g_rng = A.RuneRNG(7)
    o_state = oracle.rune_rng_state(7)
    for d in range(3):
        if logit_kind == "equal":
            logits = np.full(vocab, 1.5, np.float16)
        elif logit_kind == "two_values":
            logits = np.where(rng.random(vocab) < 0.001, 3.0, -1.0).astype(np.float16)
        else:
            logits = (rng.integers(-20, 20, vocab) * 0.5).astype(np.float16)
        t = ctx.from_numpy(logits.reshape(1, -1))
        got = A.sample_token(ctx, t, gcfg, g_rng, [])
        want, o_state = oracle.sample_token_f16(logits, ocfg, o_state, [], [])
        assert got == want, (d, got, want)
        assert g_rng.state == o_state, d
