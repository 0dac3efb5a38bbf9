"""aesir_attn_gqa_decode_static, the allocation-free variant of aesir_attn_gqa_decode: through the
C ABI, its output equals the context entry point's bit for bit on two calls in a row (the second
with a smaller input, so stale partials of the first call are in the static scratch), and both
match the CPU oracle's flash_attention_gqa within tolerance. Sizes beyond the static scratch are
rejected before any launch."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def A():
    import aesir_hip

    return aesir_hip


def _case(A, ctx, rng, S, hd, nq, nkv):
    kvd = hd * nkv
    q = (rng.standard_normal((1, nq * hd)) * 0.5).astype(np.float16)
    k = rng.standard_normal((S, kvd)).astype(np.float16)
    v = rng.standard_normal((S, kvd)).astype(np.float16)
    tq, tk, tv = ctx.from_numpy(q), ctx.from_numpy(k), ctx.from_numpy(v)
    garbage = np.full((1, nq * hd), np.nan, np.float16)
    out_ctx, out_static = ctx.from_numpy(garbage), ctx.from_numpy(garbage)
    return (q, k, v), (tq, tk, tv), out_ctx, out_static


def _call_static(A, ctx, tq, tk, tv, out, S, hd, nq, nkv):
    stream = A._L.aesir_ctx_stream(ctx.h)
    return A._L.aesir_attn_gqa_decode_static(stream, tq.ptr, 1, tk.ptr, tk.cols, tv.ptr, tv.cols, out.ptr, 1, S, hd,
                                             nq, nkv)


@pytest.mark.parametrize("shapes", [((2048, 128, 32, 8), (300, 64, 8, 2)), ((4096, 128, 32, 8), (65, 40, 6, 3))])
def test_static_attention_matches_context_entry_point(A, oracle, shapes):
    rng = np.random.default_rng(17)
    with A.Context(512 << 20) as ctx:
        for S, hd, nq, nkv in shapes:  # the second call is smaller than the first
            (q, k, v), (tq, tk, tv), out_ctx, out_static = _case(A, ctx, rng, S, hd, nq, nkv)
            A.flash_attention_gqa(ctx, tq, tk, tv, out_ctx, S, hd, nq, nkv)
            rc = _call_static(A, ctx, tq, tk, tv, out_static, S, hd, nq, nkv)
            assert rc == 0, A.last_error()
            ctx.synchronize()
            a, b = out_ctx.numpy(), out_static.numpy()
            assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), (S, hd, nq, nkv)
            ref = oracle.attn_gqa(q, k, v, np.zeros_like(q), S, hd, nq, nkv)
            err = np.abs(b.astype(np.float64) - ref.astype(np.float64))
            assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref.astype(np.float64))), (S, hd, nq, nkv)


def test_static_attention_rejects_sizes_beyond_its_scratch(A):
    with A.Context(64 << 20) as ctx:
        t = ctx.tensor(1, 256)
        stream = A._L.aesir_ctx_stream(ctx.h)
        # 4096 heads x (256 + 2) floats with one split exceed the 2^20-float static scratch; the
        # call fails on the host before any launch
        rc = A._L.aesir_attn_gqa_decode_static(stream, t.ptr, 1, t.ptr, 256, t.ptr, 256, t.ptr, 1, 1, 256, 4096, 1)
        assert rc == -7 and "static scratch of 1048576 floats" in A.last_error()
        # the reference's silent no-ops stay no-ops (return 0, nothing launched)
        assert A._L.aesir_attn_gqa_decode_static(stream, t.ptr, 1, t.ptr, 256, t.ptr, 256, t.ptr, 1, 0, 256, 1, 1) == 0
        assert A._L.aesir_attn_gqa_decode_static(stream, t.ptr, 1, t.ptr, 256, t.ptr, 256, t.ptr, 1, 4, 128, 3, 2) == 0
