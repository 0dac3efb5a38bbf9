"""Batch-1 decode benchmark of the MI355X Llama F16 forward path: tok/s and achieved HBM GB/s.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--kv 2048] [--no-cpu-baseline]

Workload: Llama-3-8B shape F16, random-init N(0, 0.02) on the device, batch 1,
greedy decode with the KV cache pre-filled to --kv positions (N(0,1) f16). A step is one full
forward pass (embedding, 32 layers, output norm, lm_head, argmax) on one token, each step
consuming the previous step's argmax on the device (HIP graph replay). Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "runeforgeai-project-aesir_amd"))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
# Synthetic weights: matrices N(0, 0.02), RMSNorm weights 1 + N(0, 0.02) (the usual ones-init of a
# norm, so that logits are not flattened and greedy streams vary from token to token).
NORM_MEAN = 1.0

# Llama-3-8B shape. head_dim = 4096 / 32 = 128, kv_dim = 1024.
DIM, LAYERS, HEADS, KV_HEADS, FFN, VOCAB = 4096, 32, 32, 8, 14336, 128256
KV_DIM = DIM // HEADS * KV_HEADS

# Algorithmic HBM bytes of one decode token: every weight matrix once, norms, one embedding row,
# K+V read over L positions and written at one.
LAYER_WEIGHT_BYTES = 2 * ((DIM + 2 * KV_DIM) * DIM + DIM * DIM + 2 * FFN * DIM + DIM * FFN + 2 * DIM)
TOKEN_WEIGHT_BYTES = LAYERS * LAYER_WEIGHT_BYTES + 2 * VOCAB * DIM + 2 * DIM + 2 * DIM
KV_BYTES_PER_POS = LAYERS * 2 * KV_DIM * 2
assert TOKEN_WEIGHT_BYTES == 15_009_857_536


def token_bytes(kv_len: int) -> int:
    return TOKEN_WEIGHT_BYTES + KV_BYTES_PER_POS * kv_len + KV_BYTES_PER_POS


# Dominant kernel: fused RMSNorm + gate/up GEMV + SwiGLU of one layer.
GATE_UP_BYTES = 2 * FFN * DIM * 2 + DIM * 2 + DIM * 2 + FFN * 2


def host_cpu() -> dict:
    """The host CPU the baseline ran on: model name (/proc/cpuinfo), logical CPUs the process may
    use, and logical CPUs of the machine."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model, "nproc": len(os.sched_getaffinity(0)), "machine_cpus": os.cpu_count()}


def cpu_baseline(kv_len: int, reps: int) -> dict:
    """Times the CPU oracle (single-threaded C restatement of the reference path) on one full
    Llama-3-8B-shape decode step at KV length kv_len: embedding row, 32 layers with their own weight
    arrays (15 GB of f16, streamed from DRAM like the reference's mmap'd weights), output norm,
    lm_head and argmax. Best of `reps` steps, each a few seconds on one core."""
    from oracle import oracle as O

    cfg = O.Config(dim=DIM, n_layers=LAYERS, n_heads=HEADS, n_kv_heads=KV_HEADS, ffn=FFN, vocab=VOCAB,
                   ctx_len=kv_len + 8)
    rng = np.random.default_rng(5)
    block = (rng.standard_normal((1 << 24) + 4099, dtype=np.float32) * 0.02).astype(np.float16)
    weights = {}
    for i, (name, (r, c)) in enumerate(O.tensor_shapes(cfg).items()):
        if name == "token_embd.weight":
            weights[name] = np.zeros((r, c), np.float16)  # only one row is read
            continue
        # distinct contents per tensor: the random block tiled from a tensor-specific offset
        weights[name] = np.resize(np.roll(block, 4099 * i), r * c).reshape(r, c)
    m = O.Model(cfg, weights)
    kv = m.new_kv()
    kv.k[:] = np.resize(block, kv.k.size).reshape(kv.k.shape) * np.float16(50)
    kv.v[:] = kv.k
    toks = [1] * (kv_len + 1)
    m.forward(kv, toks, kv_len, n_layers_run=1)  # touch pages
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        m.forward(kv, toks, kv_len)
        best = min(best, time.perf_counter() - t0)
    del m, weights
    return {"value": 1.0 / best, "unit": "tok/s", "cores": 1, "kind": "port",
            "host": host_cpu(),
            "sample": (f"C oracle (restatement of the reference CPU path), one thread: one full "
                       f"Llama-3-8B-shape decode step (32 layers, distinct weights, lm_head) at KV {kv_len}, "
                       f"best of {reps}: {best:.2f} s per token"),
            "simd": bool(O.lib().ao_simd_enabled())}


COPY_BYTES = 256 << 20


def calibrate_copy():
    """One plain copy of COPY_BYTES between two device buffers (after a warm-up copy): the kernel
    whose FETCH_SIZE / WRITE_SIZE readings calibrate the counters against a known byte count."""
    import torch

    a = torch.empty(COPY_BYTES // 4, dtype=torch.int32, device="cuda").fill_(1)
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": COPY_BYTES}))


# TinyLlama-1.1B shape (dim 2048, 22 layers, 32 q / 4 kv heads, head_dim 64, ffn 5632, vocab 32000):
# the batched-prefill workload, 128 prompt positions then 256 greedy decode steps.
TL = dict(dim=2048, layers=22, heads=32, kv_heads=4, ffn=5632, vocab=32000)
TL_KVD = TL["dim"] // TL["heads"] * TL["kv_heads"]
TL_GEMM_PARAMS = TL["layers"] * ((TL["dim"] + 2 * TL_KVD) * TL["dim"] + TL["dim"] ** 2 + 3 * TL["ffn"] * TL["dim"])
TL_WEIGHT_BYTES = 2 * (TL_GEMM_PARAMS + TL["layers"] * 2 * TL["dim"] + TL["vocab"] * TL["dim"] + 2 * TL["dim"])
# Q8_0: 34 bytes per 32 weights for every matrix a prefill streams, f16 norms
TL_Q8_WEIGHT_BYTES = (TL_GEMM_PARAMS + TL["vocab"] * TL["dim"]) * 34 // 32 + 2 * (TL["layers"] * 2 * TL["dim"] + 2 * TL["dim"])
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16


def tl_weight_bytes(wtype: str) -> int:
    """Weight bytes of the TinyLlama shape stored as wtype, as TL_WEIGHT_BYTES counts them (every
    layer matrix, the norms, one vocabulary table)."""
    if wtype == "f16":
        return TL_WEIGHT_BYTES
    if wtype == "q8_0":
        return TL_Q8_WEIGHT_BYTES
    d, kvd, f, L = TL["dim"], TL_KVD, TL["ffn"], TL["layers"]
    mats = L * (qf_mat_bytes(wtype, d + 2 * kvd, d) + qf_mat_bytes(wtype, d, d) + qf_mat_bytes(wtype, 2 * f, d)
                + qf_mat_bytes(wtype, d, f))
    return mats + qf_mat_bytes(wtype, TL["vocab"], d) + 2 * (L * 2 * d + 2 * d)


def prefill_bench(A, seed: int, n_prompt: int = 128, n_decode: int = 256, reps: int = 5, wtype: str = "f16") -> dict:
    """Batched prefill of n_prompt positions on the TinyLlama shape (one chunk up to 2048 rows: MFMA
    GEMMs, or hipBLASLt from 256 rows on; wall time of the blocking aesir_prefill call, host launches
    included), then n_decode graph-replayed greedy steps. wtype q8_0: Q8_0 matrices (weights
    dequantized per fragment, or per chunk into an f16 copy for the library GEMMs); a repacked type
    (q4_0, q4_k, ...): the tiled planes, dequantized in registers by the wide-tile GEMM, or per
    chunk into the f16 copy."""
    ctx = A.Context(TL_WEIGHT_BYTES + (1 << 30))
    types = {"f16": A.GGML_F16, "q8_0": A.GGML_Q8_0, **QF_TYPES}
    m = A.Model.create(ctx, A.ModelConfig(TL["dim"], TL["layers"], TL["heads"], TL["kv_heads"], TL["ffn"],
                                          TL["vocab"], n_prompt + n_decode + 64), types[wtype])
    m.init_random(seed, 0.02, NORM_MEAN, 0.02)
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, TL["vocab"], n_prompt).tolist()
    nxt = m.prefill(prompt)  # warm-up
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        nxt = m.prefill(prompt)
        best = min(best, time.perf_counter() - t0)
    toks, dec = [], float("nan")
    if n_decode > 0:
        m.decode_loop(nxt, n_prompt, 8)  # graph capture / warm-up
        ctx.synchronize()
        t0 = time.perf_counter()
        toks, _ = m.decode_loop(nxt, n_prompt, n_decode)
        dec = time.perf_counter() - t0
    flops = 2.0 * TL_GEMM_PARAMS * n_prompt
    m.close()
    ctx.close()
    return {"workload": f"tinyllama-1.1b shape {wtype}: {n_prompt}-token batched prefill, then "
                        f"{n_decode} greedy decode steps",
            "prefill_ms": round(best * 1e3, 3), "prefill_tok_s": round(n_prompt / best, 1),
            "gemm_tflops": round(flops / best / 1e12, 2),
            "mfma_frac": round(flops / best / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
            "weight_gbs": round(tl_weight_bytes(wtype) / best / 1e9, 1),
            "decode_tok_s": round(n_decode / dec, 1) if n_decode > 0 else None, "first_tokens": [nxt] + toks[:3]}


def q8_mat_bytes(rows: int, cols: int) -> int:
    """Q8_0 matrix in HBM: int8 quants plus one f16 scale per 32 weights (34 bytes per block)."""
    return rows * cols + rows * (cols // 32) * 2


Q8_LAYER_BYTES = (q8_mat_bytes(DIM + 2 * KV_DIM, DIM) + q8_mat_bytes(DIM, DIM) + q8_mat_bytes(2 * FFN, DIM)
                  + q8_mat_bytes(DIM, FFN) + 2 * 2 * DIM)
Q8_TOKEN_WEIGHT_BYTES = LAYERS * Q8_LAYER_BYTES + q8_mat_bytes(VOCAB, DIM) + 2 * DIM + q8_mat_bytes(1, DIM)
Q8_GATE_UP_BYTES = q8_mat_bytes(2 * FFN, DIM) + DIM * 2 + DIM * 2 + FFN * 2


REPLAY_CHECK = True  # --no-replay-check clears it (profiler runs that trace eager launches only)


def replay_check(m, kv: int, toks: list, use_graph: bool, n: int = 16):
    """Correctness evidence for a timed run, outside the timed region: the first n steps are run
    again from the same position and token with the other launch mode (eager launches after a
    graph-replayed run). The KV rows they rewrite are the ones the timed steps wrote, so the same
    tokens must come out. None when REPLAY_CHECK is off."""
    if not REPLAY_CHECK:
        return None
    n = min(n, len(toks))
    other, _ = m.decode_loop(1, kv, n, use_graph=not use_graph)
    return {"mode": "eager" if use_graph else "graph", "steps": n, "identical": other == toks[:n],
            "distinct_tokens": len(set(toks))}


def q8_bench(A, seed: int, kv: int, steps: int, warmup: int, kernel_iters: int, use_graph: bool = True) -> dict:
    """Batch-1 greedy decode of the Llama-3-8B shape with Q8_0 matrices (GGUF block_q8_0 data
    repacked as int8 quants + f16 scales; random quants, scales for weights of std 0.02), KV cache
    pre-filled to kv positions; same step structure as the F16 decode (graph replay unless
    use_graph is False)."""
    ctx_len = kv + max(steps, warmup) + 64
    # (+ the f16 copy of the largest layer matrix that long-chunk prefills dequantize into)
    well = int(Q8_TOKEN_WEIGHT_BYTES + q8_mat_bytes(VOCAB - 1, DIM) + 2 * LAYERS * ctx_len * KV_DIM * 2
               + 2 * 2 * FFN * DIM + (512 << 20))
    ctx = A.Context(well)
    m = A.Model.create(ctx, A.ModelConfig(DIM, LAYERS, HEADS, KV_HEADS, FFN, VOCAB, ctx_len), A.GGML_Q8_0)
    m.init_random(seed, 0.02, NORM_MEAN, 0.02)
    m.fill_kv_random(kv, seed=seed + 1)
    m.decode_loop(1, kv, warmup, use_graph=use_graph)
    ctx.synchronize()
    t0 = time.perf_counter()
    toks, event_ms = m.decode_loop(1, kv, steps, use_graph=use_graph)
    ctx.synchronize()
    wall = time.perf_counter() - t0
    tok_s = steps / wall
    mean_kv = kv + (steps - 1) / 2.0 + 1
    step_bytes = Q8_TOKEN_WEIGHT_BYTES + KV_BYTES_PER_POS * mean_kv + KV_BYTES_PER_POS
    check = replay_check(m, kv, toks, use_graph)
    kt = m.kernel_times(kv, iters=kernel_iters)
    gu_ms = kt["gate_up_swiglu"]
    m.close()
    ctx.close()
    return {"workload": f"llama3-8b-shape q8_0 batch-1 greedy decode, kv {kv}", "value": round(tok_s, 2),
            "unit": "tok/s", "steps": steps, "ms_per_step": round(wall * 1e3 / steps, 4),
            "dtype": "q8_0 weights (f16(q*d)), f16 activations, f32 accumulate",
            "step_hbm": {"bytes_per_token": int(step_bytes), "achieved_gbs": round(step_bytes * tok_s / 1e9, 1),
                         "frac": round(step_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4),
                         "event_ms_per_step": round(event_ms / steps, 4)},
            "gate_up_swiglu": {"avg_launch_ms": round(gu_ms, 5), "bytes_per_launch": Q8_GATE_UP_BYTES,
                               "achieved_gbs": round(Q8_GATE_UP_BYTES / (gu_ms * 1e-3) / 1e9, 1),
                               "frac": round(Q8_GATE_UP_BYTES / (gu_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
            "kernel_ms": {k: round(v, 5) for k, v in kt.items()}, "tokens_head": toks[:8], "replay_check": check}


# Repacked matrices in HBM (records of 16 weights): 4-bit nibbles (Q2_K / Q3_K values included),
# the 5-bit types' fifth-bit plane, Q6_K's 2-bit high plane, and the per-block scale planes.
QF_TYPES = {"q4_0": 2, "q4_1": 3, "q5_0": 6, "q5_1": 7, "q2_k": 10, "q3_k": 11, "q4_k": 12, "q5_k": 13, "q6_k": 14}


def qf_mat_bytes(kind: str, rows: int, cols: int) -> int:
    per_row = cols // 4 if kind in ("q2_k", "q3_k") else cols // 2  # crumb or nibble plane
    if kind in ("q5_0", "q5_1", "q5_k", "q3_k"):
        per_row += cols // 8  # fifth (Q3_K: third) bits
    if kind in ("q4_0", "q5_0", "q4_k", "q5_k"):
        per_row += cols // 32 * 2  # f16 d, or the (scale, min) bytes
    if kind in ("q4_1", "q5_1"):
        per_row += cols // 32 * 4  # f16 (d, m)
    if kind in ("q4_k", "q5_k"):
        per_row += cols // 256 * 4  # f16 (d, dmin)
    if kind in ("q2_k", "q3_k"):
        per_row += cols // 16 + cols // 256 * (4 if kind == "q2_k" else 2)  # a scale byte per 16, d (dmin)
    if kind == "q6_k":
        per_row += cols // 4 + cols // 16 + cols // 256 * 2
    return rows * per_row


def qf_token_bytes(kind: str) -> int:
    layer = (qf_mat_bytes(kind, DIM + 2 * KV_DIM, DIM) + qf_mat_bytes(kind, DIM, DIM) + qf_mat_bytes(kind, 2 * FFN, DIM)
             + qf_mat_bytes(kind, DIM, FFN) + 2 * 2 * DIM)
    return LAYERS * layer + qf_mat_bytes(kind, VOCAB, DIM) + 2 * DIM + qf_mat_bytes(kind, 1, DIM)


# llama.cpp's Q4_K_M / Q5_K_M recipes for a Llama: Q4_K (Q5_K) matrices, Q6_K for output and for
# attn_v / ffn_down of the first and last eighth of the layers and every third layer between. A
# layer whose V is Q6_K stores its Q/K/V matrix in two parts (Q and K in Q4_K / Q5_K, V in Q6_K)
# that one two-part GEMV launch reads.
MIXES = {"q4_k_m": "q4_k", "q5_k_m": "q5_k"}


def q4_k_m_more_bits(l: int) -> bool:
    return l < LAYERS // 8 or l >= 7 * LAYERS // 8 or (l - LAYERS // 8) % 3 == 2


def k_m_types(kind: str) -> dict:
    base = QF_TYPES[MIXES[kind]]
    t = {"token_embd.weight": base, "output.weight": 14}
    for l in range(LAYERS):
        for b in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"):
            t[f"blk.{l}.{b}.weight"] = 14 if b in ("attn_v", "ffn_down") and q4_k_m_more_bits(l) else base
    return t


def stored_mat_bytes(kind: str, rows: int, cols: int) -> int:
    if kind == "f16":
        return rows * cols * 2
    return q8_mat_bytes(rows, cols) if kind == "q8_0" else qf_mat_bytes(kind, rows, cols)


def layer_storage(kind: str, l: int) -> tuple:
    """Stored types of layer l's (q and k, v, o, gate/up, down) matrices."""
    if kind not in MIXES:
        return (kind,) * 5
    base, more = MIXES[kind], q4_k_m_more_bits(l)
    return (base, "q6_k" if more else base, base, base, "q6_k" if more else base)


# GGML block (weights, bytes) of each type as a GGUF file holds it (ggml's block_q*_K layouts).
GGUF_BLOCKS = {"f16": (1, 2), "q8_0": (32, 34), "q4_0": (32, 18), "q4_1": (32, 20), "q5_0": (32, 22),
               "q5_1": (32, 24), "q2_k": (256, 84), "q3_k": (256, 110), "q4_k": (256, 144),
               "q5_k": (256, 176), "q6_k": (256, 210)}


def gguf_mat_bytes(kind: str, rows: int, cols: int) -> int:
    n, b = GGUF_BLOCKS[kind]
    return rows * (cols // n) * b


def quant_token_bytes(kind: str, mat_bytes=stored_mat_bytes) -> int:
    """Algorithmic weight bytes of one decode token as stored (or, with gguf_mat_bytes, as the
    GGUF file holds them): every matrix once, norms, one embedding row."""
    embd, out = (MIXES[kind], "q6_k") if kind in MIXES else (kind, kind)
    total = mat_bytes(out, VOCAB, DIM) + 2 * DIM + mat_bytes(embd, 1, DIM)
    for l in range(LAYERS):
        qk, v, o, gu, down = layer_storage(kind, l)
        total += (mat_bytes(qk, DIM + KV_DIM, DIM) + mat_bytes(v, KV_DIM, DIM) + mat_bytes(o, DIM, DIM)
                  + mat_bytes(gu, 2 * FFN, DIM) + mat_bytes(down, DIM, FFN) + 2 * 2 * DIM)
    return total


assert all(quant_token_bytes(k) == qf_token_bytes(k) for k in QF_TYPES)
# the default run's quantized decode lines (--quant-only runs every kind)
QUANT_KINDS = ["q4_0", "q4_k", "q5_k", "q6_k", "q4_k_m", "q5_k_m"]
ALL_QUANT_KINDS = list(QF_TYPES) + list(MIXES)


def quant_bench(A, kind: str, seed: int, kv: int, steps: int, warmup: int, kernel_iters: int,
                use_graph: bool = True) -> dict:
    """Batch-1 greedy decode of the Llama-3-8B shape with matrices of one repacked type (Q4_0,
    Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K), or the Q4_K_M / Q5_K_M mixes with Q6_K (random records and
    scales for weights of std 0.02; f16 for the fused matrices a mix stores so), KV cache pre-filled
    to kv positions; same step structure and timing as the F16 decode."""
    ctx_len = kv + max(steps, warmup) + 64
    well = int(quant_token_bytes(kind) + stored_mat_bytes("q6_k", VOCAB, DIM) + 2 * LAYERS * ctx_len * KV_DIM * 2
               + 2 * 2 * FFN * DIM + (512 << 20))
    ctx = A.Context(well)
    cfg = A.ModelConfig(DIM, LAYERS, HEADS, KV_HEADS, FFN, VOCAB, ctx_len)
    if kind in MIXES:
        m = A.Model.create_mixed(ctx, cfg, k_m_types(kind))
    else:
        m = A.Model.create(ctx, cfg, QF_TYPES[kind])
    m.init_random(seed, 0.02, NORM_MEAN, 0.02)
    m.fill_kv_random(kv, seed=seed + 1)
    m.decode_loop(1, kv, warmup, use_graph=use_graph)
    ctx.synchronize()
    t0 = time.perf_counter()
    toks, event_ms = m.decode_loop(1, kv, steps, use_graph=use_graph)
    ctx.synchronize()
    wall = time.perf_counter() - t0
    tok_s = steps / wall
    mean_kv = kv + (steps - 1) / 2.0 + 1
    step_bytes = quant_token_bytes(kind) + KV_BYTES_PER_POS * mean_kv + KV_BYTES_PER_POS
    # the same token with every matrix at its GGUF size (Q2_K / Q3_K are stored wider, as 4-bit planes)
    gguf_bytes = quant_token_bytes(kind, gguf_mat_bytes) + KV_BYTES_PER_POS * mean_kv + KV_BYTES_PER_POS
    check = replay_check(m, kv, toks, use_graph)
    kt = m.kernel_times(kv, iters=kernel_iters)
    gu_ms = kt["gate_up_swiglu"]
    gu_kind = layer_storage(kind, 0)[3]  # the same in every layer
    gu_bytes = stored_mat_bytes(gu_kind, 2 * FFN, DIM) + DIM * 2 + DIM * 2 + FFN * 2
    m.close()
    ctx.close()
    dtype = (f"{MIXES[kind]} / q6_k weights (Q/K/V in two parts where V is q6_k)" if kind in MIXES else f"{kind} weights")
    return {"workload": f"llama3-8b-shape {kind} batch-1 greedy decode, kv {kv}", "value": round(tok_s, 2),
            "unit": "tok/s", "steps": steps, "ms_per_step": round(wall * 1e3 / steps, 4),
            "dtype": f"{dtype}, f16 activations, f32 accumulate",
            "step_hbm": {"bytes_per_token": int(step_bytes), "achieved_gbs": round(step_bytes * tok_s / 1e9, 1),
                         "frac": round(step_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4),
                         "event_ms_per_step": round(event_ms / steps, 4)},
            "step_hbm_gguf": {"bytes_per_token": int(gguf_bytes),
                              "frac": round(gguf_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4)},
            "gate_up_swiglu": {"avg_launch_ms": round(gu_ms, 5), "bytes_per_launch": gu_bytes,
                               "achieved_gbs": round(gu_bytes / (gu_ms * 1e-3) / 1e9, 1),
                               "frac": round(gu_bytes / (gu_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
            "kernel_ms": {k: round(v, 5) for k, v in kt.items()}, "tokens_head": toks[:8], "replay_check": check}


def sampler_bench(A, seed: int, reps: int = 50) -> dict:
    """aesir_sample_token (sample_token_from_logits on the device) over Llama-3's 128256 f16 logits
    with 256 context tokens: wall time per blocking call (host round trip included) for the greedy
    branch, a top-k 40 / top-p 0.95 / temperature 0.8 / repetition 1.1 draw, a full-vocabulary
    temperature-1 draw, and top-p 0.9 at temperature 0.9 without top-k (the truncation's two
    running sums over the whole vocabulary)."""
    rng = np.random.default_rng(seed)
    ctx = A.Context(64 << 20)
    logits = ctx.from_numpy((rng.standard_normal((1, VOCAB)) * 2.0).astype(np.float16))
    context = rng.integers(0, VOCAB, 256).tolist()
    cfgs = {"greedy_us": A.SamplerConfig(temperature=0.0),
            "topk_topp_us": A.SamplerConfig(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1),
            "full_vocab_us": A.SamplerConfig(temperature=1.0),
            "topp_only_us": A.SamplerConfig(temperature=0.9, top_p=0.9)}
    out = {"workload": f"sample_token_from_logits over {VOCAB} f16 logits, 256 context tokens"}
    r = A.RuneRNG(seed)
    for name, cfg in cfgs.items():
        for _ in range(3):
            A.sample_token(ctx, logits, cfg, r, context)
        t0 = time.perf_counter()
        for _ in range(reps):
            A.sample_token(ctx, logits, cfg, r, context)
        out[name] = round((time.perf_counter() - t0) / reps * 1e6, 1)
    ctx.close()
    return out


def kv_sweep_bench(seed: int, steps: int, warmup: int, kvs=(512, 8192, 32768)) -> dict:
    """The F16 decode of the headline at the other KV lengths of the Llama-3-8B config, each
    measured as the headline is: in a fresh process (a child started with this file's headline
    options only: the same steps and warm-up), on a model whose context length is kv + steps + warmup + 64, the cache pre-filled
    to kv, decoding from that position."""
    import subprocess

    out = {"workload": "llama3-8b-shape f16 batch-1 greedy decode (graph), KV pre-filled N(0,1); "
                       "each length in its own process"}
    for kv in kvs:
        cmd = [sys.executable, os.path.abspath(__file__), "--kv", str(kv), "--steps", str(steps), "--warmup",
               str(warmup), "--seed", str(seed), "--no-sweep", "--no-micro", "--no-prefill", "--no-q8",
               "--no-quant", "--no-cpu-baseline"]
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
        if r.returncode != 0:
            raise RuntimeError(f"kv_sweep child for KV {kv} failed ({r.returncode}): {r.stderr[-2000:]}")
        d = json.loads(r.stdout.strip().splitlines()[-1])
        h = d["step_hbm"]
        out[f"kv{kv}"] = {"tok_s": d["value"], "ms_per_step": d["ms_per_step"], "bytes_per_token": h["bytes_per_token"],
                          "achieved_gbs": h["achieved_gbs"], "frac": h["frac"],
                          "attention_us": round(d["kernel_ms"]["attention"] * 1e3, 2)}
    return out


def graph_replay_ms(A, ctx, fn, n: int) -> float:
    """HIP-event time of one replay of a graph holding fn(0) .. fn(n - 1), captured on the context
    stream (thread-local capture mode; the graph is replayed once untimed first)."""
    import ctypes as C

    hip = C.CDLL("libamdhip64.so")
    stream = C.c_void_p(A._L.aesir_ctx_stream(ctx.h))
    graph, exe = C.c_void_p(), C.c_void_p()

    def ok(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: hipError {rc}")

    ok(hip.hipStreamBeginCapture(stream, 1), "hipStreamBeginCapture")
    try:
        for i in range(n):
            fn(i)
    finally:
        ok(hip.hipStreamEndCapture(stream, C.byref(graph)), "hipStreamEndCapture")
    try:
        ok(hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0), "hipGraphInstantiate")
        ok(hip.hipGraphLaunch(exe, stream), "hipGraphLaunch")
        ctx.synchronize()
        ctx.timer_start()
        ok(hip.hipGraphLaunch(exe, stream), "hipGraphLaunch")
        return ctx.timer_stop()
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)


def micro_bench(A, seed: int, iters: int = 64, copies: int = 16, eager: bool = False) -> dict:
    """The kernel micro-suite (GEMV 4096 x 4096, RMSNorm, RoPE, argmax) and the Q8_0 GGUF-block matvec on the
    Llama-3-8B FFN shapes, through the C-ABI
    ops. Weight-sized operands rotate through `copies` buffers (more than the 256 MB MALL) so every
    call reads HBM; time per call is the HIP-event time of a graph replay of `iters` back-to-back
    calls on the context stream (argmax returns its index to the host, so its figure is a blocking
    round trip timed from the host loop; the Q8_0 lines also give the host-loop time per call).
    eager: every op timed from the host loop instead (for profiler runs that trace eager launches
    only)."""
    rng = np.random.default_rng(seed)
    ctx = A.Context(int(copies * (DIM * DIM * 2 + 1_835_008 * 34) + (512 << 20)))
    out = {}

    def host_timed(fn, n=iters):
        fn(0)
        ctx.synchronize()
        ctx.timer_start()
        for i in range(n):
            fn(i)
        return ctx.timer_stop() / n

    def timed(fn, n=iters):
        """Device time per call: the n calls are captured into one HIP graph on the context stream
        and the replay is timed with HIP events, so the Python loop's per-call overhead (which a
        C or Mojo caller does not pay) cannot starve the GPU. The first call runs eagerly outside
        the capture (it builds any cached table the op uses)."""
        if eager:
            return host_timed(fn, n)
        fn(0)
        ctx.synchronize()
        return graph_replay_ms(A, ctx, fn, n) / n

    def rate(name, us, nbytes):
        out[name] = {"us": round(us, 2), "bytes": int(nbytes), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}

    w = (rng.standard_normal((DIM, DIM)) * 0.02).astype(np.float16)
    ws = [ctx.from_numpy(w) for _ in range(copies)]
    x = ctx.from_numpy(rng.standard_normal((1, DIM)).astype(np.float16))
    y = ctx.tensor(1, DIM)
    rate("gemv_4096x4096", timed(lambda i: A.gemm_f16(ctx, x, ws[i % copies], y)) * 1e3, DIM * DIM * 2 + 4 * DIM)
    nw = ctx.from_numpy((1.0 + 0.02 * rng.standard_normal(DIM)).astype(np.float16))
    for rows in (1, 64):
        t = ctx.from_numpy(rng.standard_normal((rows, DIM)).astype(np.float16))
        rate(f"rmsnorm_{rows}x4096", timed(lambda i: A.rmsnorm(ctx, t, nw, 1e-5)) * 1e3, 2 * rows * DIM * 2 + DIM * 2)
    q = ctx.from_numpy(rng.standard_normal((4096, HEADS * 128)).astype(np.float16))
    k = ctx.from_numpy(rng.standard_normal((4096, KV_HEADS * 128)).astype(np.float16))
    rate("rope_q4096x4096_k4096x1024", timed(lambda i: A.apply_rope(ctx, q, k, 0, 128, 10000.0)) * 1e3,
         2 * 2 * 4096 * (HEADS + KV_HEADS) * 128)
    lg = ctx.from_numpy(rng.standard_normal((1, VOCAB)).astype(np.float16))
    rate("argmax_128256_blocking", host_timed(lambda i: A.argmax(ctx, lg)) * 1e3, VOCAB * 2)
    off = ctx.offset
    for n, kk in ((14336, 4096), (4096, 14336)):
        ctx.synchronize()
        ctx.reset(off)
        qq = rng.integers(-127, 128, size=(n, kk), dtype=np.int8)
        dd = rng.uniform(0.001, 0.02, size=(n, kk // 32)).astype(np.float16)
        blocks = A.Q8_0Tensor.from_parts(dd, qq).blocks.reshape(1, -1)
        bufs = [ctx.tensor(1, blocks.size, np.uint8).upload(blocks) for _ in range(copies)]
        xf = ctx.from_numpy(rng.standard_normal((1, kk)).astype(np.float32), np.float32)
        yf = ctx.tensor(1, n, np.float32)
        fn = lambda i: A.q8_0_matvec_f32(ctx, bufs[i % copies].ptr, n, kk, xf, yf)
        rate(f"q8_0_matvec_{n}x{kk}", timed(fn) * 1e3, blocks.size + 4 * kk + 4 * n)
        out[f"q8_0_matvec_{n}x{kk}"]["host_loop_us"] = round(host_timed(fn) * 1e3, 2)
    ctx.close()
    return out


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by its copy-kernel calibration factor), or None."""
    path = os.path.join(REPO, "profiles", "pmc_gate_up_swiglu_llama3_8b.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--kv", type=int, default=2048, help="KV length at the start of the timed steps")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--kernel-iters", type=int, default=5)
    ap.add_argument("--cpu-reps", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true", help="launch kernels one by one instead of graph replay")
    ap.add_argument("--no-replay-check", action="store_true",
                    help="skip re-running the timed steps in the other launch mode (for profiler runs that "
                         "trace eager launches only)")
    ap.add_argument("--no-prefill", action="store_true", help="skip the TinyLlama batched-prefill measurement")
    ap.add_argument("--prefill-only", action="store_true", help="run only the TinyLlama prefill measurement")
    ap.add_argument("--prefill-type", default="f16",
                    help="weight type of --prefill-only: f16, q8_0 or a repacked type (q4_0, q4_k, ...)")
    ap.add_argument("--prefill-decode-steps", type=int, default=256,
                    help="greedy decode steps after the prefill in --prefill-only runs (0: none)")
    ap.add_argument("--prefill-prompt", type=int, default=128,
                    help="prompt positions of --prefill-only runs (one chunk up to 2048)")
    ap.add_argument("--no-q8", action="store_true", help="skip the Q8_0-weight decode measurement")
    ap.add_argument("--no-sweep", action="store_true", help="skip the decode at KV 512 / 8192 / 32768")
    ap.add_argument("--no-micro", action="store_true", help="skip the kernel micro-suite and the Q8_0 matvec")
    ap.add_argument("--q8-only", action="store_true", help="run only the Q8_0-weight decode measurement")
    ap.add_argument("--sampler-only", action="store_true", help="run only the sampler timings")
    ap.add_argument("--no-quant", action="store_true", help="skip the quantized-weight decode measurements")
    ap.add_argument("--quant-only", action="store_true", help="run only the quantized-weight decode measurements, every type and mix")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain 256 MiB device-to-device copy (the FETCH_SIZE / WRITE_SIZE calibration "
                         "of the HBM traffic figure) and exit")
    args = ap.parse_args()
    if args.calibrate_copy:
        calibrate_copy()
        return
    global REPLAY_CHECK
    REPLAY_CHECK = not args.no_replay_check

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only (the decode path is single-GPU; multi-GPU tensor "
              "parallelism is a design, not an implementation). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import aesir_hip as A

    if args.prefill_only:
        print(json.dumps({"prefill": prefill_bench(A, args.seed, n_prompt=args.prefill_prompt,
                                                   n_decode=args.prefill_decode_steps, wtype=args.prefill_type)}))
        return
    if args.quant_only:
        print(json.dumps({"quant": {k: quant_bench(A, k, args.seed, args.kv, args.steps, args.warmup, args.kernel_iters,
                                                   not args.eager) for k in ALL_QUANT_KINDS}}))
        return
    if args.sampler_only:
        print(json.dumps({"sampler": sampler_bench(A, args.seed)}))
        return
    if args.q8_only:
        q = q8_bench(A, args.seed, args.kv, args.steps, args.warmup, args.kernel_iters, not args.eager)
        q["prefill"] = prefill_bench(A, args.seed, n_decode=min(64, args.prefill_decode_steps), wtype="q8_0")
        print(json.dumps({"q8_0": q}))
        return

    ctx_len = args.kv + max(args.steps, args.warmup) + 64
    # arena: all weights (the whole embedding table, not the one row a token reads), the KV cache
    # and 512 MiB for the decode and prefill workspaces
    model_bytes = TOKEN_WEIGHT_BYTES - 2 * DIM + 2 * VOCAB * DIM
    well = int(model_bytes + 2 * LAYERS * ctx_len * KV_DIM * 2 + (512 << 20))
    ctx = A.Context(well)
    info = ctx.device_info()
    m = A.Model.create(ctx, A.ModelConfig(DIM, LAYERS, HEADS, KV_HEADS, FFN, VOCAB, ctx_len))
    m.init_random(args.seed, 0.02, NORM_MEAN, 0.02)
    m.fill_kv_random(args.kv, seed=args.seed + 1)
    use_graph = not args.eager

    # warm-up (graph capture happens here), then the timed steps from the same KV length
    m.decode_loop(1, args.kv, args.warmup, use_graph=use_graph)
    ctx.synchronize()
    t0 = time.perf_counter()
    toks, event_ms = m.decode_loop(1, args.kv, args.steps, use_graph=use_graph)
    ctx.synchronize()
    wall = time.perf_counter() - t0

    tok_s = args.steps / wall
    ms_per_step = wall * 1e3 / args.steps
    mean_kv = args.kv + (args.steps - 1) / 2.0 + 1
    step_bytes = TOKEN_WEIGHT_BYTES + KV_BYTES_PER_POS * mean_kv + KV_BYTES_PER_POS

    check = replay_check(m, args.kv, toks, use_graph)
    kt = m.kernel_times(args.kv, iters=args.kernel_iters)
    gu_ms = kt["gate_up_swiglu"]
    gu_gbs = GATE_UP_BYTES / (gu_ms * 1e-3) / 1e9

    out = {
        "metric": "batch-1 decode tok/s + achieved HBM GB/s (% of peak), Llama-3-8B-shape F16",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 (f32 accumulate)",
        "data": "synthetic: random-init N(0,0.02) weights and 1 + N(0,0.02) norm weights generated on device, KV pre-filled N(0,1)",
        "config": {"workload": "llama3-8b-shape f16 batch-1 greedy decode", "kv_len": args.kv,
                   "dim": DIM, "layers": LAYERS, "heads": HEADS, "kv_heads": KV_HEADS, "ffn": FFN,
                   "vocab": VOCAB, "graph": use_graph, "device": info["arch"], "cu": info["cu_count"]},
        "step_hbm": {"bytes_per_token": int(step_bytes), "achieved_gbs": round(step_bytes * tok_s / 1e9, 1),
                     "frac": round(step_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4),
                     "event_ms_per_step": round(event_ms / args.steps, 4)},
        "roofline": {"bound": "hbm", "kernel": "gate_up_swiglu (rmsnorm + [2x14336x4096] GEMV + SwiGLU)",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "avg_launch_ms": round(gu_ms, 5), "bytes_per_launch": GATE_UP_BYTES},
        "kernel_ms": {k: round(v, 5) for k, v in kt.items()},
        "tokens_head": toks[:8],
        "replay_check": check,
    }
    m.close()
    ctx.close()
    if not args.no_sweep:
        out["kv_sweep"] = kv_sweep_bench(args.seed, args.steps, args.warmup)
    if not args.no_micro:
        out["micro"] = micro_bench(A, args.seed, eager=args.eager)
    if not args.no_prefill:
        out["prefill"] = prefill_bench(A, args.seed)
        # a 1024-token prompt (one chunk)
        lp = prefill_bench(A, args.seed, n_prompt=1024, n_decode=0)
        out["prefill"]["prompt_1024"] = {"prefill_ms": lp["prefill_ms"], "prefill_tok_s": lp["prefill_tok_s"],
                                         "gemm_tflops": lp["gemm_tflops"]}
    out["sampler"] = sampler_bench(A, args.seed)
    if not args.no_q8:
        out["q8_0"] = q8_bench(A, args.seed, args.kv, args.steps, args.warmup, args.kernel_iters, use_graph)
        out["q8_0"]["prefill"] = prefill_bench(A, args.seed, n_decode=64, wtype="q8_0")
        lp = prefill_bench(A, args.seed, n_prompt=1024, n_decode=0, wtype="q8_0")
        out["q8_0"]["prefill"]["prompt_1024"] = {"prefill_ms": lp["prefill_ms"], "prefill_tok_s": lp["prefill_tok_s"]}
    if not args.no_quant:
        out["quant"] = {k: quant_bench(A, k, args.seed, args.kv, args.steps, args.warmup, args.kernel_iters, use_graph)
                        for k in QUANT_KINDS}
        for k in ("q4_0", "q4_k"):  # the TinyLlama prefill with these weights (matrix-core GEMM on the planes)
            if k in out["quant"]:
                out["quant"][k]["prefill"] = prefill_bench(A, args.seed, n_decode=64, wtype=k)
                # a 1024-token prompt (one chunk: matrices dequantized to f16 for the library GEMMs)
                lp = prefill_bench(A, args.seed, n_prompt=1024, n_decode=0, wtype=k)
                out["quant"][k]["prefill"]["prompt_1024"] = {"prefill_ms": lp["prefill_ms"],
                                                             "prefill_tok_s": lp["prefill_tok_s"]}
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.kv, args.cpu_reps)
        out["cpu_baseline"]["value"] = round(out["cpu_baseline"]["value"], 4)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out))


if __name__ == "__main__":
    main()
