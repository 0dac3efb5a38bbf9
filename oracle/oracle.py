"""ctypes wrapper over liboracle.so, the CPU restatement of the reference F16 Llama path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker. The product library never imports this module.

Arrays are numpy: f16 tensors are np.float16 (bit-identical to the C side's uint16_t).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

P = C.c_void_p
I64 = C.c_int64


class OracleError(RuntimeError):
    pass


def build() -> str:
    """Compiles liboracle.so with the committed Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.ao_last_error.restype = C.c_char_p
        L.ao_f32_to_f16.restype = C.c_uint16
        L.ao_f32_to_f16.argtypes = [C.c_float]
        L.ao_f16_to_f32.restype = C.c_float
        L.ao_f16_to_f32.argtypes = [C.c_uint16]
        L.ao_f32_to_f16_array.argtypes = [P, P, I64]
        L.ao_f16_to_f32_array.argtypes = [P, P, I64]
        L.ao_gemm_f16.argtypes = [P, I64, I64, P, I64, I64, P, I64, I64]
        L.ao_rmsnorm_f16.argtypes = [P, I64, I64, P, I64, C.c_float]
        L.ao_rope_f16.argtypes = [P, I64, I64, P, I64, I64, I64, I64, C.c_float]
        L.ao_attn_gqa.argtypes = [P, I64, P, I64, P, I64, P, I64, I64, I64, I64, I64]
        L.ao_attn_gqa.restype = None
        L.ao_silu_f16.argtypes = [P, I64]
        L.ao_silu_f16.restype = None
        L.ao_mul_f16.argtypes = [P, P, I64]
        L.ao_mul_f16.restype = None
        L.ao_residual_add_f16.argtypes = [P, P, I64]
        L.ao_residual_add_f16.restype = None
        L.ao_argmax_f16.argtypes = [P, I64]
        L.ao_argmax_f16.restype = I64
        L.ao_greedy_sample_f16.argtypes = [P, I64, P, I64]
        L.ao_greedy_sample_f16.restype = I64
        L.ao_gemm_q8_0.argtypes = [P, I64, I64, P, I64, P, I64, I64]
        L.ao_dequantize_q8_0.argtypes = [P, P, I64]
        L.ao_dequantize_q8_0.restype = None
        L.ao_gemm_q4_0.argtypes = [P, I64, I64, P, I64, P, I64, I64]
        L.ao_dequantize_q4_0.argtypes = [P, P, I64]
        L.ao_dequantize_q4_0.restype = None
        L.ao_dequantize_q4_k.argtypes = [P, P, I64]
        L.ao_dequantize_q4_k.restype = None
        L.ao_dequantize_q6_k.argtypes = [P, P, I64]
        L.ao_dequantize_q6_k.restype = None
        L.ao_dequantize_q4_k_f16.argtypes = [P, P, I64]
        L.ao_dequantize_q4_k_f16.restype = None
        L.ao_dequantize_q6_k_f16.argtypes = [P, P, I64]
        L.ao_dequantize_q6_k_f16.restype = None
        L.ao_dequantize_legacy.argtypes = [C.c_int, P, P, I64]
        L.ao_gemm_legacy.argtypes = [C.c_int, P, I64, I64, P, I64, P, I64, I64]
        L.ao_dequantize_kquant.argtypes = [C.c_int, P, P, I64]
        L.ao_dequantize_kquant_f16.argtypes = [C.c_int, P, P, I64]
        L.ao_kv_append.argtypes = [P, I64, I64, P, I64, P, I64]
        L.ao_kv_slice.argtypes = [P, I64, I64, P, P]
        L.ao_forward_scratch_elems.argtypes = [P]
        L.ao_forward_scratch_elems.restype = I64
        L.ao_forward_pass.argtypes = [P, P, P, I64, I64, P, P, P]
        L.ao_forward_partial.argtypes = [P, P, P, I64, I64, I64, P, P, P]
        L.ao_generation_stop_reason.argtypes = [I64, I64, I64, I64, P, I64, I64, I64]
        L.ao_generate.argtypes = [P, P, P, I64, I64, I64, P, I64, P, P, P, P, P]
        L.ao_rune_rng_next.argtypes = [P]
        L.ao_rune_rng_next.restype = C.c_uint64
        L.ao_rune_rng_next_float32.argtypes = [P]
        L.ao_rune_rng_next_float32.restype = C.c_float
        L.ao_sample_candidates_f16.argtypes = [P, I64, P, P, I64, P, I64, P, P]
        L.ao_sample_candidates_f16.restype = I64
        L.ao_sample_token_f16.argtypes = [P, I64, P, P, I64, P, I64, P]
        L.ao_sample_token_f16.restype = I64
        L.ao_fill_normal_f16.argtypes = [P, I64, C.c_uint64, C.c_uint64, C.c_float, C.c_float]
        L.ao_fill_normal_f16.restype = None
        L.ao_fill_normal_f32.argtypes = [P, I64, C.c_uint64, C.c_uint64, C.c_float, C.c_float]
        L.ao_fill_normal_f32.restype = None
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _check(rc: int):
    if rc != 0:
        raise OracleError(lib().ao_last_error().decode())


def last_error() -> str:
    return lib().ao_last_error().decode()


# ---------------------------------------------------------------- conversions

def f32_to_f16_bits(x: float) -> int:
    return int(lib().ao_f32_to_f16(float(x)))


def to_f16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.float16)
    lib().ao_f32_to_f16_array(_ptr(a), _ptr(out), a.size)
    return out


def to_f32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().ao_f16_to_f32_array(_ptr(a), _ptr(out), a.size)
    return out


# ---------------------------------------------------------------- kernels

def _f16(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    assert a.dtype == np.float16, a.dtype
    return a


def gemm_f16(A, B, c_shape=None) -> np.ndarray:
    A, B = _f16(A), _f16(B)
    ar, ac = A.shape
    br, bc = B.shape
    cr, cc = c_shape if c_shape is not None else (ar, br)
    Cm = np.zeros((max(cr, 1), max(cc, 1)), dtype=np.float16)
    _check(lib().ao_gemm_f16(_ptr(A), ar, ac, _ptr(B), br, bc, _ptr(Cm), cr, cc))
    return Cm


def rmsnorm_f16(T, w, eps=1e-5) -> np.ndarray:
    T = _f16(T).copy()
    w = _f16(w)
    rows, cols = T.shape
    _check(lib().ao_rmsnorm_f16(_ptr(T), rows, cols, _ptr(w), w.size, eps))
    return T


def rope_f16(Q, K, start_pos, head_dim, theta=10000.0):
    Q = _f16(Q).copy()
    K = _f16(K).copy()
    _check(lib().ao_rope_f16(_ptr(Q), Q.shape[0], Q.shape[1], _ptr(K), K.shape[0], K.shape[1],
                             start_pos, head_dim, theta))
    return Q, K


def attn_gqa(q, keys, values, out, seq_len, head_dim, nq, nkv) -> np.ndarray:
    """flash_attention_gqa; `out` is copied and returned (untouched on the no-op paths)."""
    q, keys, values = _f16(q), _f16(keys), _f16(values)
    out = _f16(out).copy()
    lib().ao_attn_gqa(_ptr(q), q.shape[0], _ptr(keys), keys.shape[1], _ptr(values), values.shape[1],
                      _ptr(out), out.shape[0], seq_len, head_dim, nq, nkv)
    return out


def silu_f16(T) -> np.ndarray:
    T = _f16(T).copy()
    lib().ao_silu_f16(_ptr(T), T.size)
    return T


def mul_f16(up, gate) -> np.ndarray:
    up = _f16(up).copy()
    gate = _f16(gate)
    lib().ao_mul_f16(_ptr(up), _ptr(gate), up.size)
    return up


def residual_add_f16(x, r) -> np.ndarray:
    x = _f16(x).copy()
    r = _f16(r)
    lib().ao_residual_add_f16(_ptr(x), _ptr(r), x.size)
    return x


def argmax_f16(logits) -> int:
    logits = _f16(logits)
    return int(lib().ao_argmax_f16(_ptr(logits), logits.size))


def greedy_sample_f16(logits, suppress=()) -> int:
    logits = _f16(logits)
    s = np.ascontiguousarray(np.array(list(suppress) or [0], dtype=np.int64))
    return int(lib().ao_greedy_sample_f16(_ptr(logits), logits.size, _ptr(s), len(suppress)))


class SamplerConfig(C.Structure):
    """Parameters of sample_token_from_logits (sampler.mojo:217-230)."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int64), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repetition_penalty", C.c_float), ("frequency_penalty", C.c_float),
                ("presence_penalty", C.c_float)]

    def __init__(self, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repetition_penalty=1.0,
                 frequency_penalty=0.0, presence_penalty=0.0):
        super().__init__(temperature, top_k, top_p, min_p, repetition_penalty, frequency_penalty, presence_penalty)


def _i64(seq):
    return np.ascontiguousarray(np.array(list(seq) or [0], dtype=np.int64))


def rune_rng_state(seed: int) -> int:
    """RuneRNG.__init__ (sampler.mojo:25-29): seed 0 maps to 0x9E3779B97F4A7C15."""
    return seed if seed != 0 else 0x9E3779B97F4A7C15


def rune_rng_next_float32(state: int):
    st = C.c_uint64(state)
    v = lib().ao_rune_rng_next_float32(C.byref(st))
    return float(v), st.value


def sample_candidates_f16(logits, cfg: SamplerConfig, context=(), suppress=()):
    """Candidate ids and f32 logits after the mask, penalties, temperature and truncations."""
    logits = _f16(logits)
    ids = np.zeros(logits.size, np.int64)
    lg = np.zeros(logits.size, np.float32)
    c, sp = _i64(context), _i64(suppress)
    n = lib().ao_sample_candidates_f16(_ptr(logits), logits.size, C.byref(cfg), _ptr(c), len(context), _ptr(sp),
                                       len(suppress), _ptr(ids), _ptr(lg))
    return ids[:n], lg[:n]


def sample_token_f16(logits, cfg: SamplerConfig, rng_state: int, context=(), suppress=()):
    """sample_token_from_logits: (token, new RuneRNG state)."""
    logits = _f16(logits)
    c, sp = _i64(context), _i64(suppress)
    st = C.c_uint64(rng_state)
    tok = lib().ao_sample_token_f16(_ptr(logits), logits.size, C.byref(cfg), _ptr(c), len(context), _ptr(sp),
                                    len(suppress), C.byref(st))
    return int(tok), st.value


def gemm_q8_0(A, blocks, n_rows) -> np.ndarray:
    A = _f16(A)
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    Cm = np.zeros((A.shape[0], n_rows), dtype=np.float16)
    _check(lib().ao_gemm_q8_0(_ptr(A), A.shape[0], A.shape[1], _ptr(blocks), n_rows, _ptr(Cm),
                              A.shape[0], n_rows))
    return Cm


def gemm_q4_0(A, blocks, n_rows) -> np.ndarray:
    A = _f16(A)
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    Cm = np.zeros((A.shape[0], n_rows), dtype=np.float16)
    _check(lib().ao_gemm_q4_0(_ptr(A), A.shape[0], A.shape[1], _ptr(blocks), n_rows, _ptr(Cm),
                              A.shape[0], n_rows))
    return Cm


def dequantize_q4_0(blocks, n_blocks) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n_blocks * 32, dtype=np.float16)
    lib().ao_dequantize_q4_0(_ptr(blocks), _ptr(out), n_blocks)
    return out


def dequantize_q4_k(blocks, n_blocks) -> np.ndarray:
    """GGML block_q4_K super-blocks (144 bytes) -> f32 weights."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n_blocks * 256, dtype=np.float32)
    lib().ao_dequantize_q4_k(_ptr(blocks), _ptr(out), n_blocks)
    return out


def dequantize_q6_k(blocks, n_blocks) -> np.ndarray:
    """GGML block_q6_K super-blocks (210 bytes) -> f32 weights."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n_blocks * 256, dtype=np.float32)
    lib().ao_dequantize_q6_k(_ptr(blocks), _ptr(out), n_blocks)
    return out


def dequantize_q4_k_f16(blocks, n_blocks) -> np.ndarray:
    """GGML block_q4_K super-blocks -> the library's f16 weights f16(f16(d sc) q - f16(dmin m))."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n_blocks * 256, dtype=np.float16)
    lib().ao_dequantize_q4_k_f16(_ptr(blocks), _ptr(out), n_blocks)
    return out


def dequantize_q6_k_f16(blocks, n_blocks) -> np.ndarray:
    """GGML block_q6_K super-blocks -> the library's f16 weights f16(f16(d sc) (q - 32))."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n_blocks * 256, dtype=np.float16)
    lib().ao_dequantize_q6_k_f16(_ptr(blocks), _ptr(out), n_blocks)
    return out


def dequantize_q8_0(blocks, n_blocks) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n_blocks * 32, dtype=np.float16)
    lib().ao_dequantize_q8_0(_ptr(blocks), _ptr(out), n_blocks)
    return out


LEGACY_TYPES = {"q4_1": 3, "q5_0": 6, "q5_1": 7}
KQUANT_TYPES = {"q2_k": 10, "q3_k": 11, "q5_k": 13}


def dequantize_legacy(kind: str, blocks, n_blocks) -> np.ndarray:
    """GGUF block_q4_1 / _q5_0 / _q5_1 -> the reference's f16 weights (dequantize_q4_1 / _q5_0 /
    _q5_1, core/compute.mojo:282-340)."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n_blocks * 32, dtype=np.float16)
    _check(lib().ao_dequantize_legacy(LEGACY_TYPES[kind], _ptr(blocks), _ptr(out), n_blocks))
    return out


def gemm_legacy(kind: str, A, blocks, n_rows) -> np.ndarray:
    """gemm_q4_1 / _q5_0 / _q5_1 (core/compute.mojo:914-1036) on GGUF blocks."""
    A = _f16(A)
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    Cm = np.zeros((A.shape[0], n_rows), dtype=np.float16)
    _check(lib().ao_gemm_legacy(LEGACY_TYPES[kind], _ptr(A), A.shape[0], A.shape[1], _ptr(blocks), n_rows, _ptr(Cm),
                                A.shape[0], n_rows))
    return Cm


def dequantize_kquant(kind: str, blocks, n_blocks) -> np.ndarray:
    """GGML block_q2_K / _q3_K / _q5_K super-blocks -> GGML's f32 weights."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n_blocks * 256, dtype=np.float32)
    _check(lib().ao_dequantize_kquant(KQUANT_TYPES[kind], _ptr(blocks), _ptr(out), n_blocks))
    return out


def dequantize_kquant_f16(kind: str, blocks, n_blocks) -> np.ndarray:
    """GGML block_q2_K / _q3_K / _q5_K super-blocks -> the library's f16 weights."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n_blocks * 256, dtype=np.float16)
    _check(lib().ao_dequantize_kquant_f16(KQUANT_TYPES[kind], _ptr(blocks), _ptr(out), n_blocks))
    return out


# ---------------------------------------------------------------- KV cache

class _KV(C.Structure):
    _fields_ = [("k", P), ("v", P), ("max_seq", I64), ("kv_dim", I64), ("num_layers", I64)]


class KVCache:
    """KVCache over numpy buffers (mimir_well.mojo:434-521)."""

    def __init__(self, max_seq, kv_dim, num_layers):
        self.k = np.zeros((num_layers * max_seq, kv_dim), dtype=np.float16)
        self.v = np.zeros((num_layers * max_seq, kv_dim), dtype=np.float16)
        self.s = _KV(self.k.ctypes.data, self.v.ctypes.data, max_seq, kv_dim, num_layers)

    def append(self, layer, pos, key, val):
        key, val = _f16(key), _f16(val)
        _check(lib().ao_kv_append(C.byref(self.s), layer, pos, _ptr(key), key.size, _ptr(val), val.size))

    def slices(self, layer, seq_len):
        kp, vp = C.c_void_p(), C.c_void_p()
        _check(lib().ao_kv_slice(C.byref(self.s), layer, seq_len, C.byref(kp), C.byref(vp)))
        base = self.k.ctypes.data
        row0 = (kp.value - base) // (2 * self.s.kv_dim)
        return self.k[row0:row0 + seq_len], self.v[row0:row0 + seq_len]


# ---------------------------------------------------------------- model

class _Cfg(C.Structure):
    _fields_ = [("dim", I64), ("n_layers", I64), ("n_heads", I64), ("n_kv_heads", I64), ("ffn", I64),
                ("vocab", I64), ("ctx_len", I64), ("eps", C.c_float), ("theta", C.c_float)]


class _Model(C.Structure):
    _fields_ = [("cfg", _Cfg), ("token_embd", P), ("output_norm", P), ("output", P),
                ("attn_norm", P), ("wq", P), ("wk", P), ("wv", P), ("wo", P), ("ffn_norm", P),
                ("w_gate", P), ("w_up", P), ("w_down", P)]


@dataclass
class Config:
    dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    ffn: int
    vocab: int
    ctx_len: int
    eps: float = 1e-5
    theta: float = 10000.0

    @property
    def head_dim(self) -> int:
        return self.dim // self.n_heads

    @property
    def kv_dim(self) -> int:
        return self.head_dim * self.n_kv_heads


# Tensor order used by the counter-based synthetic generator: stream id = index in this list
# for the globals, then 100 + 16*layer + slot for per-layer tensors.
LAYER_TENSORS = ["attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm",
                 "ffn_gate", "ffn_up", "ffn_down"]
GLOBAL_TENSORS = ["token_embd", "output_norm", "output"]


def tensor_stream(name: str) -> int:
    name = name[: -len(".weight")] if name.endswith(".weight") else name
    if name in GLOBAL_TENSORS:
        return GLOBAL_TENSORS.index(name)
    _, layer, base = name.split(".")[:3]
    return 100 + 16 * int(layer) + LAYER_TENSORS.index(base)


def tensor_shapes(cfg: Config) -> dict:
    d, kv, f, V = cfg.dim, cfg.kv_dim, cfg.ffn, cfg.vocab
    shapes = {"token_embd.weight": (V, d), "output_norm.weight": (1, d), "output.weight": (V, d)}
    per = {"attn_norm": (1, d), "attn_q": (d, d), "attn_k": (kv, d), "attn_v": (kv, d),
           "attn_output": (d, d), "ffn_norm": (1, d), "ffn_gate": (f, d), "ffn_up": (f, d),
           "ffn_down": (d, f)}
    for l in range(cfg.n_layers):
        for k, s in per.items():
            shapes[f"blk.{l}.{k}.weight"] = s
    return shapes


def fill_normal_f16(n: int, seed: int, stream: int, mean=0.0, std=0.02) -> np.ndarray:
    out = np.empty(n, dtype=np.float16)
    lib().ao_fill_normal_f16(_ptr(out), n, seed, stream, mean, std)
    return out


def fill_normal_f32(n: int, seed: int, stream: int, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().ao_fill_normal_f32(_ptr(out), n, seed, stream, mean, std)
    return out


def synthetic_weights(cfg: Config, seed: int, std=0.02, norm_mean=0.0, norm_std=0.02) -> dict:
    """Seeded random-init weights, every tensor N(0, std) -> f16 (norm tensors N(norm_mean,
    norm_std)). Norm tensors are rounded to f16 here, as the reference's F32->F16 load does."""
    w = {}
    for name, (r, c) in tensor_shapes(cfg).items():
        base = name.split(".")[-2]
        s = tensor_stream(name)
        if base.endswith("norm"):
            w[name] = fill_normal_f16(r * c, seed, s, norm_mean, norm_std).reshape(r, c)
        else:
            w[name] = fill_normal_f16(r * c, seed, s, 0.0, std).reshape(r, c)
    return w


def prompt_tokens(n: int, vocab: int, seed: int) -> list:
    """Uniform token IDs from RuneRNG (sampler.mojo:17-43)."""
    st = C.c_uint64(seed if seed != 0 else 0x9E3779B97F4A7C15)
    return [int(lib().ao_rune_rng_next(C.byref(st)) % vocab) for _ in range(n)]


class Model:
    """Holds numpy weights and the ao_model view of them."""

    def __init__(self, cfg: Config, weights: dict):
        self.cfg = cfg
        self.w = {k: np.ascontiguousarray(v, dtype=np.float16) for k, v in weights.items()}
        L = cfg.n_layers
        self._arrs = {}
        for key, base in [("attn_norm", "attn_norm"), ("wq", "attn_q"), ("wk", "attn_k"),
                          ("wv", "attn_v"), ("wo", "attn_output"), ("ffn_norm", "ffn_norm"),
                          ("w_gate", "ffn_gate"), ("w_up", "ffn_up"), ("w_down", "ffn_down")]:
            arr = (P * L)(*[self.w[f"blk.{l}.{base}.weight"].ctypes.data for l in range(L)])
            self._arrs[key] = arr
        self.s = _Model(_Cfg(cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.ffn, cfg.vocab,
                             cfg.ctx_len, cfg.eps, cfg.theta),
                        self.w["token_embd.weight"].ctypes.data, self.w["output_norm.weight"].ctypes.data,
                        self.w["output.weight"].ctypes.data,
                        *[C.cast(self._arrs[k], P) for k in ["attn_norm", "wq", "wk", "wv", "wo",
                                                             "ffn_norm", "w_gate", "w_up", "w_down"]])
        self.scratch = np.zeros(lib().ao_forward_scratch_elems(C.byref(self.s.cfg)), dtype=np.float16)

    def new_kv(self) -> KVCache:
        return KVCache(self.cfg.ctx_len, self.cfg.kv_dim, self.cfg.n_layers)

    def forward(self, kv: KVCache, tokens, start_pos, n_layers_run=None):
        toks = np.ascontiguousarray(np.array(tokens, dtype=np.int64))
        logits = np.zeros(self.cfg.vocab, dtype=np.float16)
        nxt = C.c_int64()
        n_run = self.cfg.n_layers if n_layers_run is None else n_layers_run
        _check(lib().ao_forward_partial(C.byref(self.s), C.byref(kv.s), _ptr(toks), toks.size, start_pos,
                                        n_run, _ptr(self.scratch), _ptr(logits), C.byref(nxt)))
        return int(nxt.value), logits

    def generate(self, prompt, max_new, eos=-1, stop_tokens=()):
        kv = self.new_kv()
        p = np.ascontiguousarray(np.array(prompt, dtype=np.int64))
        st = np.ascontiguousarray(np.array(list(stop_tokens) or [0], dtype=np.int64))
        out = np.zeros(max_new + 1, dtype=np.int64)
        n_out = C.c_int64()
        reason = C.c_int32(-1)
        logits = np.zeros(self.cfg.vocab, dtype=np.float16)
        _check(lib().ao_generate(C.byref(self.s), C.byref(kv.s), _ptr(p), p.size, max_new, eos, _ptr(st),
                                 len(stop_tokens), _ptr(self.scratch), _ptr(out), C.byref(n_out),
                                 C.byref(reason), _ptr(logits)))
        return [int(t) for t in out[: n_out.value]], STOP_REASONS[reason.value], logits


STOP_REASONS = {0: "eos", 1: "stop_token", 2: "length", 3: "context_exhausted"}


def stop_reason(token, eos, generated_count, max_new, stop_tokens, next_position, ctx_len) -> str:
    st = np.ascontiguousarray(np.array(list(stop_tokens) or [0], dtype=np.int64))
    r = lib().ao_generation_stop_reason(token, eos, generated_count, max_new, _ptr(st), len(stop_tokens),
                                        next_position, ctx_len)
    return STOP_REASONS.get(r, "")


TINY = Config(dim=64, n_layers=5, n_heads=8, n_kv_heads=4, ffn=172, vocab=512, ctx_len=512)
TINYLLAMA = Config(dim=2048, n_layers=22, n_heads=32, n_kv_heads=4, ffn=5632, vocab=32000, ctx_len=2048)
LLAMA3_8B = Config(dim=4096, n_layers=32, n_heads=32, n_kv_heads=8, ffn=14336, vocab=128256,
                   ctx_len=32768, theta=10000.0)
