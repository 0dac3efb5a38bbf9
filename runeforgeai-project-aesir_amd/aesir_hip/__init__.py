"""Python host-side binding of libaesir_hip.so (ctypes over the C ABI in include/aesir_hip.h).

It mirrors the reference's kernel-call and engine API (aesir_engine/core/compute.mojo,
core/mimir_well.mojo, core/inference.mojo, aesir.mojo) with the same names, argument meaning and
error behaviour: failing calls raise AesirError carrying the library's message, which is the
reference's own text where the reference raises. Tensors are device buffers carved from the
context's HBM arena (the MimirWell); numpy arrays are the host side.

There is no fallback: if libaesir_hip.so is missing, importing this module raises.
"""
from __future__ import annotations

import ctypes as C
import os
import weakref
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libaesir_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"libaesir_hip.so not built at {LIB_PATH}: run python runeforgeai-project-aesir_amd/build.py")

_L = C.CDLL(LIB_PATH)

P = C.c_void_p
I64 = C.c_int64
I32 = C.c_int32
F32 = C.c_float


class AesirError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class _ModelConfig(C.Structure):
    _fields_ = [("dim", I64), ("n_layers", I64), ("n_heads", I64), ("n_kv_heads", I64), ("ffn", I64),
                ("vocab", I64), ("ctx_len", I64), ("rms_eps", F32), ("rope_theta", F32),
                ("bos_token_id", I64), ("eos_token_id", I64)]


class _GenConfig(C.Structure):
    _fields_ = [("max_new_tokens", I64), ("stop_tokens", P), ("n_stop_tokens", I64), ("batched_prefill", I32)]


def _sig(name, args, res=I32):
    f = getattr(_L, name)
    f.argtypes = args
    f.restype = res
    return f


_sig("aesir_last_error", [], C.c_char_p)
_sig("aesir_abi_version", [])
_sig("aesir_ctx_create", [I32, I64, C.POINTER(P)])
_sig("aesir_ctx_destroy", [P])
_sig("aesir_ctx_synchronize", [P])
_sig("aesir_ctx_stream", [P], P)
_sig("aesir_ctx_device_info", [P, C.c_char_p, I32, C.POINTER(I32), C.POINTER(I64)])
_sig("aesir_well_allocate", [P, I64, C.POINTER(P)])
_sig("aesir_well_reset", [P, I64])
_sig("aesir_well_offset", [P], I64)
_sig("aesir_well_capacity", [P], I64)
_sig("aesir_memcpy_h2d", [P, P, P, I64])
_sig("aesir_memcpy_d2h", [P, P, P, I64])
_sig("aesir_memcpy_d2d", [P, P, P, I64])
_sig("aesir_timer_start", [P])
_sig("aesir_timer_stop", [P, C.POINTER(F32)])
_sig("aesir_gemm_f16", [P, P, I64, I64, P, I64, I64, P, I64, I64])
_sig("aesir_rmsnorm_f16", [P, P, I64, I64, P, I64, F32])
_sig("aesir_rope_f16", [P, P, I64, I64, P, I64, I64, I64, I64, F32])
_sig("aesir_attn_gqa_decode", [P, P, I64, P, I64, P, I64, P, I64, I64, I64, I64, I64])
_sig("aesir_attn_gqa_decode_static", [P, P, I64, P, I64, P, I64, P, I64, I64, I64, I64, I64])
_sig("aesir_silu_f16", [P, P, I64])
_sig("aesir_swiglu_f16", [P, P, P, I64])
_sig("aesir_residual_add_f16", [P, P, P, I64])
_sig("aesir_embed_f16", [P, P, I64, I64, I64, P])
_sig("aesir_argmax_f16", [P, P, I64, C.POINTER(I64)])
_sig("aesir_gemm_q8_0", [P, P, I64, I64, P, I64, P, I64, I64])
_sig("aesir_gemm_quant", [P, P, I64, I64, P, I32, I64, P, I64, I64])
_sig("aesir_q8_0_matvec_f32", [P, P, I64, I64, P, P])
_sig("aesir_kv_create", [P, I64, I64, I64, C.POINTER(P)])
_sig("aesir_kv_destroy", [P])
_sig("aesir_kv_append", [P, P, I64, I64, P, I64, P, I64])
_sig("aesir_kv_k_slice", [P, I64, I64, C.POINTER(P)])
_sig("aesir_kv_v_slice", [P, I64, I64, C.POINTER(P)])
_sig("aesir_model_create", [P, C.POINTER(_ModelConfig), C.POINTER(P)])
_sig("aesir_model_create_typed", [P, C.POINTER(_ModelConfig), I32, C.POINTER(P)])
_sig("aesir_model_create_mixed", [P, C.POINTER(_ModelConfig), P, I64, C.POINTER(P)])
_sig("aesir_model_weight_type", [P])
_sig("aesir_model_tensor_type", [P, C.c_char_p])
_sig("aesir_model_destroy", [P])
_sig("aesir_model_get_config", [P, C.POINTER(_ModelConfig)])
_sig("aesir_model_set_tensor", [P, C.c_char_p, P, I64, I64, I32])
_sig("aesir_model_get_tensor", [P, C.c_char_p, P, I64])
_sig("aesir_model_init_random", [P, C.c_uint64, F32, F32, F32])
_sig("aesir_model_load_gguf", [P, C.c_char_p, I64, C.POINTER(P)])
_sig("aesir_gguf_inspect", [C.c_char_p, C.POINTER(_ModelConfig), C.POINTER(F32)])
_sig("aesir_forward_pass", [P, P, I64, I64, C.POINTER(I64)])
_sig("aesir_forward_pass_no_cache", [P, P, I64, C.POINTER(I64)])
_sig("aesir_model_logits", [P, P])
_sig("aesir_decode_loop", [P, I64, I64, I64, I32, P, C.POINTER(F32)])
_sig("aesir_model_kernel_times", [P, I64, I32, P, I32])
_sig("aesir_prefill", [P, P, I64, I64, P])
_sig("aesir_sample_token", [P, P, I64, P, P, I64, P, I64, P, P])
_sig("aesir_rune_rng_next", [P], C.c_uint64)
_sig("aesir_model_fill_kv_random", [P, I64, C.c_uint64, F32])
_sig("aesir_generation_stop_reason", [I64, I64, I64, I64, P, I64, I64, I64])
_sig("aesir_generate", [P, P, I64, C.POINTER(_GenConfig), P, C.POINTER(I64), C.POINTER(I32)])

HEADER = os.path.join(os.path.dirname(os.path.dirname(_HERE)), "include", "aesir_hip.h")


def declared_functions(header: str = HEADER) -> list:
    """Names of every function include/aesir_hip.h declares."""
    import re

    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aesir_[a-z0-9_]+)\s*\(", text)))


def missing_exports() -> list:
    """Declared functions that the loaded library does not export (should be empty)."""
    out = []
    for name in declared_functions():
        try:
            getattr(_L, name)
        except AttributeError:
            out.append(name)
    return out


def _check(rc: int):
    if rc != 0:
        raise AesirError(rc, _L.aesir_last_error().decode())


def last_error() -> str:
    return _L.aesir_last_error().decode()


def abi_version() -> int:
    return _L.aesir_abi_version()


STOP_REASONS = {0: "eos", 1: "stop_token", 2: "length", 3: "context_exhausted"}
KERNEL_CLASSES = ["qkv_rope_kv", "attention", "o_residual", "gate_up_swiglu", "down_residual", "lm_head",
                  "argmax_finish"]


class Tensor:
    """RuneTensor view: a device pointer with (rows, cols); dtype f16 unless stated."""

    def __init__(self, ctx: "Context", ptr: int, rows: int, cols: int, dtype=np.float16):
        self.ctx, self.ptr, self.rows, self.cols, self.dtype = ctx, ptr, rows, cols, np.dtype(dtype)

    @property
    def size(self) -> int:
        return self.rows * self.cols

    @property
    def nbytes(self) -> int:
        return self.size * self.dtype.itemsize

    def numpy(self) -> np.ndarray:
        out = np.empty((self.rows, self.cols), dtype=self.dtype)
        if self.size:
            _check(_L.aesir_memcpy_d2h(self.ctx.h, out.ctypes.data, self.ptr, self.nbytes))
        return out

    def upload(self, a: np.ndarray) -> "Tensor":
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.size == self.size, (a.shape, self.rows, self.cols)
        _check(_L.aesir_memcpy_h2d(self.ctx.h, self.ptr, a.ctypes.data, self.nbytes))
        return self

    def view(self, rows: int, cols: int, offset_elems: int = 0) -> "Tensor":
        return Tensor(self.ctx, self.ptr + offset_elems * self.dtype.itemsize, rows, cols, self.dtype)


class Context:
    """One GPU, one HIP stream, one HBM arena (MimirWell, core/mimir_well.mojo:524-569)."""

    def __init__(self, well_bytes: int = 1 << 30, device: int = 0):
        h = P()
        _check(_L.aesir_ctx_create(device, int(well_bytes), C.byref(h)))
        self.h = h.value
        self._models = weakref.WeakSet()  # models hold pointers into the context: closed first

    def close(self):
        if self.h:
            for m in list(self._models):
                m.close()
            _check(_L.aesir_ctx_destroy(self.h))
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def device_info(self) -> dict:
        buf = C.create_string_buffer(64)
        cu = I32()
        hbm = I64()
        _check(_L.aesir_ctx_device_info(self.h, buf, 64, C.byref(cu), C.byref(hbm)))
        return {"arch": buf.value.decode(), "cu_count": cu.value, "hbm_bytes": hbm.value}

    def synchronize(self):
        _check(_L.aesir_ctx_synchronize(self.h))

    # ---- MimirWell
    def allocate(self, elements: int) -> int:
        p = P()
        _check(_L.aesir_well_allocate(self.h, int(elements), C.byref(p)))
        return p.value

    @property
    def offset(self) -> int:
        return _L.aesir_well_offset(self.h)

    @property
    def capacity(self) -> int:
        return _L.aesir_well_capacity(self.h)

    def reset(self, offset: int):
        _check(_L.aesir_well_reset(self.h, int(offset)))

    def tensor(self, rows: int, cols: int, dtype=np.float16) -> Tensor:
        itemsize = np.dtype(dtype).itemsize
        elems = max(1, (rows * cols * itemsize + 1) // 2)
        return Tensor(self, self.allocate(elems), rows, cols, dtype)

    def from_numpy(self, a: np.ndarray, dtype=np.float16) -> Tensor:
        a = np.asarray(a)
        rows, cols = (1, a.size) if a.ndim == 1 else a.shape
        return self.tensor(rows, cols, dtype).upload(a)

    # ---- timing (HIP events on the context stream)
    def timer_start(self):
        _check(_L.aesir_timer_start(self.h))

    def timer_stop(self) -> float:
        ms = F32()
        _check(_L.aesir_timer_stop(self.h, C.byref(ms)))
        return ms.value


# ------------------------------------------------------------------ kernel-call API

def gemm_f16(ctx: Context, A: Tensor, B: Tensor, C_: Tensor):
    """gemm_f16(A, B, C): C[m,n] = f16(sum_k A[m,k] B[n,k]) (core/compute.mojo:1751-1854)."""
    _check(_L.aesir_gemm_f16(ctx.h, A.ptr, A.rows, A.cols, B.ptr, B.rows, B.cols, C_.ptr, C_.rows, C_.cols))


def rmsnorm(ctx: Context, T: Tensor, weight: Tensor, epsilon: float = 1e-5):
    _check(_L.aesir_rmsnorm_f16(ctx.h, T.ptr, T.rows, T.cols, weight.ptr, weight.size, epsilon))


def apply_rope(ctx: Context, Q: Tensor, K: Tensor, start_pos: int, head_dim: int, theta: float = 10000.0):
    _check(_L.aesir_rope_f16(ctx.h, Q.ptr, Q.rows, Q.cols, K.ptr, K.rows, K.cols, start_pos, head_dim, theta))


def flash_attention_gqa(ctx: Context, query: Tensor, keys: Tensor, values: Tensor, output: Tensor,
                        sequence_length: int, head_dim: int, query_head_count: int, kv_head_count: int):
    _check(_L.aesir_attn_gqa_decode(ctx.h, query.ptr, query.rows, keys.ptr, keys.cols, values.ptr, values.cols,
                                    output.ptr, output.rows, sequence_length, head_dim, query_head_count,
                                    kv_head_count))


def silu(ctx: Context, T: Tensor):
    _check(_L.aesir_silu_f16(ctx.h, T.ptr, T.size))


def swiglu(ctx: Context, up: Tensor, gate: Tensor):
    _check(_L.aesir_swiglu_f16(ctx.h, up.ptr, gate.ptr, up.size))


def residual_add(ctx: Context, x: Tensor, residual: Tensor):
    _check(_L.aesir_residual_add_f16(ctx.h, x.ptr, residual.ptr, x.size))


def embed(ctx: Context, table: Tensor, token: int, x: Tensor):
    _check(_L.aesir_embed_f16(ctx.h, table.ptr, table.rows, table.cols, token, x.ptr))


def argmax(ctx: Context, logits: Tensor) -> int:
    out = I64()
    _check(_L.aesir_argmax_f16(ctx.h, logits.ptr, logits.size, C.byref(out)))
    return out.value


def gemm_q8_0(ctx: Context, A: Tensor, blocks_ptr: int, b_rows: int, C_: Tensor):
    _check(_L.aesir_gemm_q8_0(ctx.h, A.ptr, A.rows, A.cols, blocks_ptr, b_rows, C_.ptr, C_.rows, C_.cols))


def gemm_quant(ctx: Context, A: Tensor, blocks_ptr: int, ggml_type: int, b_rows: int, C_: Tensor):
    """gemm_f16's quantized branch (core/compute.mojo:1763-1800) over packed GGUF blocks on the device."""
    _check(_L.aesir_gemm_quant(ctx.h, A.ptr, A.rows, A.cols, blocks_ptr, ggml_type, b_rows, C_.ptr, C_.rows, C_.cols))


def q8_0_matvec_f32(ctx: Context, blocks_ptr: int, n_rows: int, k: int, x: Tensor, y: Tensor):
    _check(_L.aesir_q8_0_matvec_f32(ctx.h, blocks_ptr, n_rows, k, x.ptr, y.ptr))


class SamplerConfig(C.Structure):
    """sample_token_from_logits parameters (core/sampler.mojo:217-230); defaults leave every stage off
    except the draw at temperature 1."""
    _fields_ = [("temperature", F32), ("top_k", I64), ("top_p", F32), ("min_p", F32),
                ("repetition_penalty", F32), ("frequency_penalty", F32), ("presence_penalty", F32)]

    def __init__(self, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repetition_penalty=1.0,
                 frequency_penalty=0.0, presence_penalty=0.0):
        super().__init__(temperature, top_k, top_p, min_p, repetition_penalty, frequency_penalty, presence_penalty)


class RuneRNG:
    """RuneRNG (core/sampler.mojo:17-43) on the host; its state feeds sample_token."""

    def __init__(self, seed: int = 42):
        self.state = seed if seed != 0 else 0x9E3779B97F4A7C15

    def next_u64(self) -> int:
        st = C.c_uint64(self.state)
        v = _L.aesir_rune_rng_next(C.byref(st))
        self.state = st.value
        return int(v)


def sample_token(ctx: Context, logits: Tensor, cfg: SamplerConfig, rng: RuneRNG, context_tokens=(),
                 suppress_tokens=()) -> int:
    """sample_token_from_logits on the device (logits: f16 device tensor of vocab entries)."""
    c = np.ascontiguousarray(np.array(list(context_tokens) or [0], dtype=np.int64))
    sp = np.ascontiguousarray(np.array(list(suppress_tokens) or [0], dtype=np.int64))
    st = C.c_uint64(rng.state)
    tok = I64()
    _check(_L.aesir_sample_token(ctx.h, logits.ptr, logits.size, C.byref(cfg), c.ctypes.data, len(context_tokens),
                                 sp.ctypes.data, len(suppress_tokens), C.byref(st), C.byref(tok)))
    rng.state = st.value
    return tok.value


class KVCache:
    """KVCache (core/mimir_well.mojo:434-521) carved from the context's well."""

    def __init__(self, ctx: Context, max_seq_len: int, hidden_dim: int, num_layers: int = 32):
        h = P()
        _check(_L.aesir_kv_create(ctx.h, max_seq_len, hidden_dim, num_layers, C.byref(h)))
        self.ctx, self.h = ctx, h.value
        self.max_seq_len, self.hidden_dim, self.num_layers = max_seq_len, hidden_dim, num_layers

    def __del__(self):
        if getattr(self, "h", None):
            _L.aesir_kv_destroy(self.h)
            self.h = None

    def append(self, layer_idx: int, pos: int, key: Tensor, val: Tensor):
        _check(_L.aesir_kv_append(self.ctx.h, self.h, layer_idx, pos, key.ptr, key.size, val.ptr, val.size))

    def get_k_slice(self, layer_idx: int, seq_len: int) -> Tensor:
        p = P()
        _check(_L.aesir_kv_k_slice(self.h, layer_idx, seq_len, C.byref(p)))
        return Tensor(self.ctx, p.value, seq_len, self.hidden_dim)

    def get_v_slice(self, layer_idx: int, seq_len: int) -> Tensor:
        p = P()
        _check(_L.aesir_kv_v_slice(self.h, layer_idx, seq_len, C.byref(p)))
        return Tensor(self.ctx, p.value, seq_len, self.hidden_dim)


# ------------------------------------------------------------------ model / engine

@dataclass
class ModelConfig:
    dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    ffn: int
    vocab: int
    ctx_len: int
    rms_eps: float = 1e-5
    rope_theta: float = 10000.0
    bos_token_id: int = 1
    eos_token_id: int = 2

    def _c(self) -> _ModelConfig:
        return _ModelConfig(self.dim, self.n_layers, self.n_heads, self.n_kv_heads, self.ffn, self.vocab,
                            self.ctx_len, self.rms_eps, self.rope_theta, self.bos_token_id, self.eos_token_id)


GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 2, 8, 12, 14
GGML_Q4_1, GGML_Q5_0, GGML_Q5_1, GGML_Q2_K, GGML_Q3_K, GGML_Q5_K = 3, 6, 7, 10, 11, 13
WEIGHT_MIXED = -2  # aesir_model_weight_type of a model whose matrices differ in type


class QuantTensor:
    """A rows x cols matrix as the packed GGML blocks of one quantized type, in row order (the
    bytes a GGUF file holds for the tensor). Subclasses fix the type's block geometry."""

    ggml_type = -1
    block_elems = 0
    block_bytes = 0

    def __init__(self, blocks: np.ndarray, rows: int, cols: int):
        if cols % self.block_elems:
            raise ValueError(f"{type(self).__name__} rows must be a multiple of {self.block_elems} long")
        nb = rows * cols // self.block_elems
        self.blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(nb, self.block_bytes)
        self.rows, self.cols = rows, cols


class Q8_0Tensor(QuantTensor):
    """GGUF block_q8_0: rows * cols / 32 packed 34-byte blocks {f16 d; int8 qs[32]} (GGML type 8)."""

    ggml_type, block_elems, block_bytes = 8, 32, 34

    @classmethod
    def from_parts(cls, d: np.ndarray, q: np.ndarray) -> "Q8_0Tensor":
        """d: f16 scales [rows, cols/32]; q: int8 quants [rows, cols]."""
        rows, cols = q.shape
        nb = rows * cols // 32
        blocks = np.empty((nb, 34), np.uint8)
        blocks[:, :2] = np.ascontiguousarray(d, np.float16).reshape(nb).view(np.uint8).reshape(nb, 2)
        blocks[:, 2:] = np.ascontiguousarray(q, np.int8).reshape(nb, 32).view(np.uint8)
        return cls(blocks, rows, cols)

    def dequantize(self) -> np.ndarray:
        """f16(q * d) per element (the product is exact in f32, then one rounding)."""
        d = self.blocks[:, :2].copy().view(np.float16).astype(np.float32)
        q = self.blocks[:, 2:].copy().view(np.int8).astype(np.float32)
        return (q * d).astype(np.float16).reshape(self.rows, self.cols)


class Q4_0Tensor(QuantTensor):
    """GGUF block_q4_0: 18-byte blocks {f16 d; uint8 qs[16]} of 32 weights (GGML type 2); byte i
    holds element i in its low nibble and element i + 16 in its high nibble."""

    ggml_type, block_elems, block_bytes = 2, 32, 18

    @classmethod
    def from_parts(cls, d: np.ndarray, q: np.ndarray) -> "Q4_0Tensor":
        """d: f16 scales [rows, cols/32]; q: 4-bit values 0..15 [rows, cols]."""
        rows, cols = q.shape
        nb = rows * cols // 32
        qb = np.ascontiguousarray(q, np.uint8).reshape(nb, 32) & 15
        blocks = np.empty((nb, 18), np.uint8)
        blocks[:, :2] = np.ascontiguousarray(d, np.float16).reshape(nb).view(np.uint8).reshape(nb, 2)
        blocks[:, 2:] = qb[:, :16] | (qb[:, 16:] << 4)
        return cls(blocks, rows, cols)

    def dequantize(self) -> np.ndarray:
        """dequantize_q4_0 (core/compute.mojo:266-280): f16((q - 8) * d), one rounding."""
        d = self.blocks[:, :2].copy().view(np.float16).astype(np.float32)
        qs = self.blocks[:, 2:]
        q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.float32) - 8.0
        return (q * d).astype(np.float16).reshape(self.rows, self.cols)


class Q4_KTensor(QuantTensor):
    """GGUF block_q4_K: 144-byte super-blocks of 256 weights (GGML type 12):
    {f16 d; f16 dmin; uint8 scales[12]; uint8 qs[128]}, eight sub-blocks of 32 with a 6-bit scale
    and a 6-bit min each; w = d * scale * q - dmin * min."""

    ggml_type, block_elems, block_bytes = 12, 256, 144

    @classmethod
    def from_parts(cls, d, dmin, scales, mins, q) -> "Q4_KTensor":
        """d, dmin: f16 [rows, cols/256]; scales, mins: 0..63 [rows, cols/256, 8]; q: 0..15 [rows, cols]."""
        rows, cols = q.shape
        nb = rows * cols // 256
        sc = np.ascontiguousarray(scales, np.uint8).reshape(nb, 8) & 63
        mn = np.ascontiguousarray(mins, np.uint8).reshape(nb, 8) & 63
        packed = np.zeros((nb, 12), np.uint8)
        packed[:, 0:4] = sc[:, 0:4] | ((sc[:, 4:8] >> 4) << 6)
        packed[:, 4:8] = mn[:, 0:4] | ((mn[:, 4:8] >> 4) << 6)
        packed[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
        qb = np.ascontiguousarray(q, np.uint8).reshape(nb, 4, 64) & 15
        qs = (qb[:, :, :32] | (qb[:, :, 32:] << 4)).reshape(nb, 128)
        blocks = np.empty((nb, 144), np.uint8)
        blocks[:, 0:2] = np.ascontiguousarray(d, np.float16).reshape(nb).view(np.uint8).reshape(nb, 2)
        blocks[:, 2:4] = np.ascontiguousarray(dmin, np.float16).reshape(nb).view(np.uint8).reshape(nb, 2)
        blocks[:, 4:16] = packed
        blocks[:, 16:] = qs
        return cls(blocks, rows, cols)


class Q6_KTensor(QuantTensor):
    """GGUF block_q6_K: 210-byte super-blocks of 256 weights (GGML type 14):
    {uint8 ql[128]; uint8 qh[64]; int8 scales[16]; f16 d}, sixteen sub-blocks of 16 with an int8
    scale each; w = d * scale * (q - 32) for 6-bit q."""

    ggml_type, block_elems, block_bytes = 14, 256, 210

    @classmethod
    def from_parts(cls, d, scales, q) -> "Q6_KTensor":
        """d: f16 [rows, cols/256]; scales: int8 [rows, cols/256, 16]; q: 0..63 [rows, cols]."""
        rows, cols = q.shape
        nb = rows * cols // 256
        qv = (np.ascontiguousarray(q, np.uint8) & 63).reshape(nb, 2, 4, 32)  # [block, half, group, l]
        ql = np.empty((nb, 2, 64), np.uint8)
        ql[:, :, :32] = (qv[:, :, 0] & 15) | ((qv[:, :, 2] & 15) << 4)
        ql[:, :, 32:] = (qv[:, :, 1] & 15) | ((qv[:, :, 3] & 15) << 4)
        qh = (qv[:, :, 0] >> 4) | ((qv[:, :, 1] >> 4) << 2) | ((qv[:, :, 2] >> 4) << 4) | ((qv[:, :, 3] >> 4) << 6)
        blocks = np.empty((nb, 210), np.uint8)
        blocks[:, 0:128] = ql.reshape(nb, 128)
        blocks[:, 128:192] = qh.reshape(nb, 64)
        blocks[:, 192:208] = np.ascontiguousarray(scales, np.int8).reshape(nb, 16).view(np.uint8)
        blocks[:, 208:210] = np.ascontiguousarray(d, np.float16).reshape(nb).view(np.uint8).reshape(nb, 2)
        return cls(blocks, rows, cols)


def _f16_bytes(a, nb: int) -> np.ndarray:
    return np.ascontiguousarray(a, np.float16).reshape(nb).view(np.uint8).reshape(nb, 2)


def _legacy_qs(q: np.ndarray, nb: int) -> np.ndarray:
    """16 nibble bytes per 32 weights: element i low, element i + 16 high."""
    qb = np.ascontiguousarray(q, np.uint8).reshape(nb, 32) & 15
    return qb[:, :16] | (qb[:, 16:] << 4)


def _legacy_qh(q: np.ndarray, nb: int) -> np.ndarray:
    """4 bytes per 32 weights: bit i % 8 of byte i / 8 is element i's fifth bit."""
    hb = (np.ascontiguousarray(q, np.uint8).reshape(nb, 4, 8) >> 4) & 1
    return (hb << np.arange(8, dtype=np.uint8)).sum(axis=2).astype(np.uint8)


class Q4_1Tensor(QuantTensor):
    """GGUF block_q4_1: 20-byte blocks {f16 d; f16 m; uint8 qs[16]} of 32 weights (GGML type 3, the
    reference's BlockQ4_1); w = f16(f16(q d) + m)."""

    ggml_type, block_elems, block_bytes = 3, 32, 20

    @classmethod
    def from_parts(cls, d, m, q) -> "Q4_1Tensor":
        """d, m: f16 [rows, cols/32]; q: 0..15 [rows, cols]."""
        rows, cols = q.shape
        nb = rows * cols // 32
        blocks = np.empty((nb, 20), np.uint8)
        blocks[:, 0:2] = _f16_bytes(d, nb)
        blocks[:, 2:4] = _f16_bytes(m, nb)
        blocks[:, 4:] = _legacy_qs(q, nb)
        return cls(blocks, rows, cols)


class Q5_0Tensor(QuantTensor):
    """GGUF block_q5_0: 22-byte blocks {f16 d; uint8 qh[4]; uint8 qs[16]} of 32 weights (GGML type
    6, the reference's BlockQ5_0); w = f16((q - 16) d) for 5-bit q."""

    ggml_type, block_elems, block_bytes = 6, 32, 22

    @classmethod
    def from_parts(cls, d, q) -> "Q5_0Tensor":
        """d: f16 [rows, cols/32]; q: 0..31 [rows, cols]."""
        rows, cols = q.shape
        nb = rows * cols // 32
        blocks = np.empty((nb, 22), np.uint8)
        blocks[:, 0:2] = _f16_bytes(d, nb)
        blocks[:, 2:6] = _legacy_qh(q, nb)
        blocks[:, 6:] = _legacy_qs(q, nb)
        return cls(blocks, rows, cols)


class Q5_1Tensor(QuantTensor):
    """GGUF block_q5_1: 24-byte blocks {f16 d; f16 m; uint8 qh[4]; uint8 qs[16]} of 32 weights (GGML
    type 7, the reference's BlockQ5_1); w = f16(f16(q d) + m) for 5-bit q."""

    ggml_type, block_elems, block_bytes = 7, 32, 24

    @classmethod
    def from_parts(cls, d, m, q) -> "Q5_1Tensor":
        """d, m: f16 [rows, cols/32]; q: 0..31 [rows, cols]."""
        rows, cols = q.shape
        nb = rows * cols // 32
        blocks = np.empty((nb, 24), np.uint8)
        blocks[:, 0:2] = _f16_bytes(d, nb)
        blocks[:, 2:4] = _f16_bytes(m, nb)
        blocks[:, 4:8] = _legacy_qh(q, nb)
        blocks[:, 8:] = _legacy_qs(q, nb)
        return cls(blocks, rows, cols)


class Q5_KTensor(QuantTensor):
    """GGUF block_q5_K: 176-byte super-blocks of 256 weights (GGML type 13):
    {f16 d; f16 dmin; uint8 scales[12]; uint8 qh[32]; uint8 qs[128]}, Q4_K's scales and nibble
    order plus a fifth bit per weight; w = d * scale * q - dmin * min for 5-bit q."""

    ggml_type, block_elems, block_bytes = 13, 256, 176

    @classmethod
    def from_parts(cls, d, dmin, scales, mins, q) -> "Q5_KTensor":
        """d, dmin: f16 [rows, cols/256]; scales, mins: 0..63 [rows, cols/256, 8]; q: 0..31 [rows, cols]."""
        rows, cols = q.shape
        nb = rows * cols // 256
        base = Q4_KTensor.from_parts(d, dmin, scales, mins, np.ascontiguousarray(q, np.uint8) & 15).blocks
        hb = ((np.ascontiguousarray(q, np.uint8).reshape(nb, 8, 32) >> 4) & 1)  # [block, sub-block 2g + hi, l]
        qh = (hb << np.arange(8, dtype=np.uint8)[None, :, None]).sum(axis=1).astype(np.uint8)
        blocks = np.empty((nb, 176), np.uint8)
        blocks[:, 0:16] = base[:, 0:16]
        blocks[:, 16:48] = qh
        blocks[:, 48:] = base[:, 16:]
        return cls(blocks, rows, cols)


class Q2_KTensor(QuantTensor):
    """GGUF block_q2_K: 84-byte super-blocks of 256 weights (GGML type 10):
    {uint8 scales[16]; uint8 qs[64]; f16 d; f16 dmin}, sixteen sub-blocks of 16 with a 4-bit scale
    and min each; w = d * scale * q - dmin * min for 2-bit q."""

    ggml_type, block_elems, block_bytes = 10, 256, 84

    @classmethod
    def from_parts(cls, d, dmin, scales, mins, q) -> "Q2_KTensor":
        """d, dmin: f16 [rows, cols/256]; scales, mins: 0..15 [rows, cols/256, 16]; q: 0..3 [rows, cols]."""
        rows, cols = q.shape
        nb = rows * cols // 256
        qv = (np.ascontiguousarray(q, np.uint8) & 3).reshape(nb, 2, 4, 32)  # [block, half, shift, l]
        qs = (qv << (2 * np.arange(4, dtype=np.uint8))[None, None, :, None]).sum(axis=2).astype(np.uint8)
        blocks = np.empty((nb, 84), np.uint8)
        blocks[:, 0:16] = ((np.ascontiguousarray(scales, np.uint8) & 15)
                           | ((np.ascontiguousarray(mins, np.uint8) & 15) << 4)).reshape(nb, 16)
        blocks[:, 16:80] = qs.reshape(nb, 64)
        blocks[:, 80:82] = _f16_bytes(d, nb)
        blocks[:, 82:84] = _f16_bytes(dmin, nb)
        return cls(blocks, rows, cols)


class Q3_KTensor(QuantTensor):
    """GGUF block_q3_K: 110-byte super-blocks of 256 weights (GGML type 11):
    {uint8 hmask[32]; uint8 qs[64]; uint8 scales[12]; f16 d}, sixteen sub-blocks of 16 with a
    6-bit scale each (stored + 32); w = d * scale * q for q in -4..3."""

    ggml_type, block_elems, block_bytes = 11, 256, 110

    @classmethod
    def from_parts(cls, d, scales, q) -> "Q3_KTensor":
        """d: f16 [rows, cols/256]; scales: -32..31 [rows, cols/256, 16]; q: -4..3 [rows, cols]."""
        rows, cols = q.shape
        nb = rows * cols // 256
        qv = np.ascontiguousarray(q, np.int16).reshape(nb, 2, 4, 32)  # [block, half, shift, l]
        low = (qv & 3).astype(np.uint8)                                  # q + 4 when q < 0, else q
        high = (qv >= 0).astype(np.uint8)
        qs = (low << (2 * np.arange(4, dtype=np.uint8))[None, None, :, None]).sum(axis=2).astype(np.uint8)
        hm = (high << (np.arange(2)[:, None] * 4 + np.arange(4)[None, :]).astype(np.uint8)[None, :, :, None])
        hmask = hm.sum(axis=(1, 2)).astype(np.uint8)
        u = (np.ascontiguousarray(scales, np.int16).reshape(nb, 16) + 32).astype(np.uint8) & 63
        sc = np.zeros((nb, 12), np.uint8)
        sc[:, 0:8] = (u[:, 0:8] & 15) | ((u[:, 8:16] & 15) << 4)
        for j in range(16):
            sc[:, 8 + j % 4] |= (u[:, j] >> 4) << (2 * (j // 4))
        blocks = np.empty((nb, 110), np.uint8)
        blocks[:, 0:32] = hmask
        blocks[:, 32:96] = qs.reshape(nb, 64)
        blocks[:, 96:108] = sc
        blocks[:, 108:110] = _f16_bytes(d, nb)
        return cls(blocks, rows, cols)


class Model:
    """One Llama model in HBM (F16 or Q8_0 matrices): forward_pass (core/inference.mojo:424-518)
    and the generation loop (aesir.mojo:323-462)."""

    def __init__(self, ctx: Context, handle: int):
        self.ctx, self.h = ctx, handle
        ctx._models.add(self)
        c = _ModelConfig()
        _check(_L.aesir_model_get_config(self.h, C.byref(c)))
        self.cfg = ModelConfig(c.dim, c.n_layers, c.n_heads, c.n_kv_heads, c.ffn, c.vocab, c.ctx_len, c.rms_eps,
                               c.rope_theta, c.bos_token_id, c.eos_token_id)

    @classmethod
    def create(cls, ctx: Context, cfg: ModelConfig, weight_type: int = GGML_F16) -> "Model":
        h = P()
        c = cfg._c()
        if weight_type == GGML_F16:
            _check(_L.aesir_model_create(ctx.h, C.byref(c), C.byref(h)))
        else:
            _check(_L.aesir_model_create_typed(ctx.h, C.byref(c), weight_type, C.byref(h)))
        return cls(ctx, h.value)

    @classmethod
    def create_mixed(cls, ctx: Context, cfg: ModelConfig, types: dict) -> "Model":
        """A model with one type per matrix (aesir_model_create_mixed): `types` maps GGUF tensor
        names ("token_embd.weight", "blk.N.attn_v.weight", ...) to GGML types; matrices it does
        not name are F16."""
        names = ["token_embd.weight", "output.weight"] + [
            f"blk.{l}.{b}.weight" for l in range(cfg.n_layers)
            for b in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")]
        unknown = set(types) - set(names)
        if unknown:
            raise ValueError(f"not a model matrix: {sorted(unknown)[0]}")
        t = np.array([types.get(n, GGML_F16) for n in names], np.int32)
        h = P()
        c = cfg._c()
        _check(_L.aesir_model_create_mixed(ctx.h, C.byref(c), t.ctypes.data, t.size, C.byref(h)))
        return cls(ctx, h.value)

    @property
    def weight_type(self) -> int:
        return _L.aesir_model_weight_type(self.h)

    def tensor_type(self, name: str) -> int:
        """GGML type that set_tensor takes for the named tensor."""
        rc = _L.aesir_model_tensor_type(self.h, name.encode())
        if rc < 0:
            raise AesirError(rc, _L.aesir_last_error().decode())
        return rc

    @classmethod
    def load_gguf(cls, ctx: Context, path: str, ctx_len: int = 0) -> "Model":
        h = P()
        _check(_L.aesir_model_load_gguf(ctx.h, path.encode(), ctx_len, C.byref(h)))
        return cls(ctx, h.value)

    def close(self):
        if self.h:
            _L.aesir_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_tensor(self, name: str, data):
        if isinstance(data, QuantTensor):
            _check(_L.aesir_model_set_tensor(self.h, name.encode(), data.blocks.ctypes.data, data.rows, data.cols,
                                             data.ggml_type))
            return
        data = np.asarray(data)
        ggml = 0 if data.dtype == np.float32 else 1
        data = np.ascontiguousarray(data, dtype=np.float32 if ggml == 0 else np.float16)
        rows, cols = (1, data.size) if data.ndim == 1 else data.shape
        _check(_L.aesir_model_set_tensor(self.h, name.encode(), data.ctypes.data, rows, cols, ggml))

    def set_weights(self, weights: dict):
        for k, v in weights.items():
            self.set_tensor(k, v)

    def get_tensor(self, name: str, shape) -> np.ndarray:
        out = np.empty(shape, dtype=np.float16)
        _check(_L.aesir_model_get_tensor(self.h, name.encode(), out.ctypes.data, out.size))
        return out

    def init_random(self, seed: int, std: float = 0.02, norm_mean: float = 0.0, norm_std: float = 0.02):
        _check(_L.aesir_model_init_random(self.h, seed, std, norm_mean, norm_std))

    def forward_pass(self, tokens, start_pos: int) -> int:
        t = np.ascontiguousarray(np.array(tokens, dtype=np.int64))
        out = I64()
        _check(_L.aesir_forward_pass(self.h, t.ctypes.data if t.size else None, t.size, start_pos, C.byref(out)))
        return out.value

    def forward_pass_no_cache(self, tokens) -> int:
        """forward_pass without an explicit KVCache (core/inference.mojo:521-547): the last token at
        position len(tokens) - 1 over a fresh (zeroed) cache; the model's cache is cleared first."""
        t = np.ascontiguousarray(np.array(tokens, dtype=np.int64))
        out = I64()
        _check(_L.aesir_forward_pass_no_cache(self.h, t.ctypes.data if t.size else None, t.size, C.byref(out)))
        return out.value

    def prefill(self, tokens, start_pos: int = 0) -> int:
        """Batched prefill of tokens at positions start_pos..: the same KV cache and next token as
        forward_pass at each position in turn (aesir.mojo:358-374), one pass per chunk of up to 2048
        rows."""
        t = np.ascontiguousarray(np.array(tokens, dtype=np.int64))
        nxt = I64()
        _check(_L.aesir_prefill(self.h, t.ctypes.data, len(t), start_pos, C.byref(nxt)))
        return nxt.value

    def logits(self) -> np.ndarray:
        out = np.empty(self.cfg.vocab, dtype=np.float16)
        _check(_L.aesir_model_logits(self.h, out.ctypes.data))
        return out

    def decode_loop(self, token: int, start_pos: int, n_steps: int, use_graph: bool = True):
        out = np.zeros(n_steps, dtype=np.int64)
        ms = F32()
        _check(_L.aesir_decode_loop(self.h, token, start_pos, n_steps, 1 if use_graph else 0, out.ctypes.data,
                                    C.byref(ms)))
        return out.tolist(), ms.value

    def fill_kv_random(self, n_pos: int, seed: int = 1, std: float = 1.0):
        _check(_L.aesir_model_fill_kv_random(self.h, n_pos, seed, std))

    def kernel_times(self, pos: int, iters: int = 10) -> dict:
        t = np.zeros(7, dtype=np.float32)
        _check(_L.aesir_model_kernel_times(self.h, pos, iters, t.ctypes.data, 7))
        return dict(zip(KERNEL_CLASSES, t.tolist()))

    def generate(self, prompt, max_new_tokens: int, stop_tokens=(), batched_prefill: bool = False):
        p = np.ascontiguousarray(np.array(prompt, dtype=np.int64))
        st = np.ascontiguousarray(np.array(list(stop_tokens) or [0], dtype=np.int64))
        g = _GenConfig(max_new_tokens, st.ctypes.data, len(stop_tokens), 1 if batched_prefill else 0)
        out = np.zeros(max(1, max_new_tokens), dtype=np.int64)
        n = I64()
        reason = I32(-1)
        _check(_L.aesir_generate(self.h, p.ctypes.data if p.size else None, p.size, C.byref(g), out.ctypes.data,
                                 C.byref(n), C.byref(reason)))
        return out[: n.value].tolist(), STOP_REASONS[reason.value]


def gguf_inspect(path: str):
    """Validates a GGUF file without a GPU; returns (ModelConfig, rope_freq_base)."""
    c = _ModelConfig()
    fb = F32()
    _check(_L.aesir_gguf_inspect(path.encode(), C.byref(c), C.byref(fb)))
    return (ModelConfig(c.dim, c.n_layers, c.n_heads, c.n_kv_heads, c.ffn, c.vocab, c.ctx_len, c.rms_eps,
                        c.rope_theta, c.bos_token_id, c.eos_token_id), fb.value)


def generation_stop_reason(token, eos, generated_count, max_new, stop_tokens, next_position, ctx_len) -> str:
    st = np.ascontiguousarray(np.array(list(stop_tokens) or [0], dtype=np.int64))
    r = _L.aesir_generation_stop_reason(token, eos, generated_count, max_new, st.ctypes.data, len(stop_tokens),
                                        next_position, ctx_len)
    return STOP_REASONS.get(r, "")
