"""Writes the committed golden fixtures from the CPU oracle (run from the repo root):

    python tests/golden/make_golden.py

tiny_stream.npz: the tiny model (stories260K shape, random-init N(0, 0.02) from SEED), a
16-token RuneRNG prompt and the 64 greedy tokens the oracle produces, plus its last f16 logits.
micro_small.npz: small-size micro-suite outputs (GEMV, RMSNorm, RoPE, argmax) on seeded inputs.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402

SEED, PROMPT_SEED, N_NEW = 1234, 7, 64


def tiny_stream():
    cfg = O.TINY
    m = O.Model(cfg, O.synthetic_weights(cfg, SEED))
    prompt = O.prompt_tokens(16, cfg.vocab, PROMPT_SEED)
    toks, reason, logits = m.generate(prompt, N_NEW)
    assert reason == "length"
    np.savez(os.path.join(HERE, "tiny_stream.npz"), seed=np.int64(SEED), prompt=np.array(prompt, np.int64),
             n_new=np.int64(N_NEW), tokens=np.array(toks, np.int64), last_logits=logits)
    return toks


def micro_small():
    rng = np.random.default_rng(99)
    x = rng.standard_normal((1, 512)).astype(np.float16)
    w = (rng.standard_normal((96, 512)) * 0.02).astype(np.float16)
    rx = rng.standard_normal((4, 512)).astype(np.float16)
    rw = (1 + 0.1 * rng.standard_normal(512)).astype(np.float16)
    q = rng.standard_normal((16, 4 * 128)).astype(np.float16)
    k = rng.standard_normal((16, 2 * 128)).astype(np.float16)
    rq, rk = O.rope_f16(q, k, 100, 128)
    logits = rng.standard_normal(4099).astype(np.float16)
    np.savez(os.path.join(HERE, "micro_small.npz"), gemv_x=x, gemv_w=w, gemv_y=O.gemm_f16(x, w),
             rms_x=rx, rms_w=rw, rms_y=O.rmsnorm_f16(rx, rw, 1e-5), rope_q=q, rope_k=k, rope_q_out=rq,
             rope_k_out=rk, argmax_logits=logits, argmax_index=np.int64(O.argmax_f16(logits)))


if __name__ == "__main__":
    print(tiny_stream())
    micro_small()
