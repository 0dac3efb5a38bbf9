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


def test_static_attention_under_graph_capture(A):
    """Code under HIP graph capture, the caller this entry point is for: after one eager call on
    the device (which resolves the scratch address; the first call on a device must not be inside
    a capture), a captured call replays bit for bit like the eager one, also when an eager call
    with other inputs has rewritten the shared static scratch between replays."""
    hip = C.CDLL("libamdhip64.so")
    for f in ("hipStreamCreate", "hipStreamSynchronize", "hipStreamBeginCapture", "hipStreamEndCapture",
              "hipGraphInstantiate", "hipGraphLaunch", "hipGraphExecDestroy", "hipGraphDestroy", "hipStreamDestroy"):
        getattr(hip, f).restype = C.c_int
    rng = np.random.default_rng(23)
    S, hd, nq, nkv = 2048, 128, 32, 8
    with A.Context(512 << 20) as ctx:
        (q, k, v), (tq, tk, tv), out_ref, out_graph = _case(A, ctx, rng, S, hd, nq, nkv)
        _, (oq, ok_, ov), out_other, _ = _case(A, ctx, rng, 3000, hd, nq, nkv)
        stream = C.c_void_p()
        assert hip.hipStreamCreate(C.byref(stream)) == 0

        def static(tq_, tk_, tv_, out, S_):
            return A._L.aesir_attn_gqa_decode_static(stream, tq_.ptr, 1, tk_.ptr, tk_.cols, tv_.ptr, tv_.cols,
                                                     out.ptr, 1, S_, hd, nq, nkv)

        assert static(tq, tk, tv, out_ref, S) == 0, A.last_error()  # eager call (also the warm-up)
        assert hip.hipStreamSynchronize(stream) == 0
        ref = out_ref.numpy()
        graph, exe = C.c_void_p(), C.c_void_p()
        assert hip.hipStreamBeginCapture(stream, 1) == 0  # thread-local capture mode
        rc = static(tq, tk, tv, out_graph, S)
        assert hip.hipStreamEndCapture(stream, C.byref(graph)) == 0
        assert rc == 0, A.last_error()
        assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
        try:
            for _ in range(3):
                out_graph.upload(np.full((1, nq * hd), np.nan, np.float16))
                assert static(oq, ok_, ov, out_other, 3000) == 0  # eager work on the same scratch
                assert hip.hipGraphLaunch(exe, stream) == 0
                assert hip.hipStreamSynchronize(stream) == 0
                assert np.array_equal(out_graph.numpy().view(np.uint16), ref.view(np.uint16))
        finally:
            hip.hipGraphExecDestroy(exe)
            hip.hipGraphDestroy(graph)
            hip.hipStreamDestroy(stream)
