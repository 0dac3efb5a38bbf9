"""Minimal GGUF v3 writer for test fixtures (the gguf Python package is not installed).

Writes the subset the reference loader reads (loader/gguf.mojo:322-377): general.architecture,
llama.* dimensions, rms epsilon, tokenizer arrays and special ids, general.alignment, then a
tensor table and 32-byte aligned data. Tensors are given in GGUF order (rows x cols, cols
fastest: ne0 = cols, ne1 = rows).
"""
from __future__ import annotations

import struct

import numpy as np

T_UINT32, T_INT32, T_FLOAT32, T_BOOL, T_STRING, T_ARRAY = 4, 5, 6, 7, 8, 9


def _s(b: bytearray, text: str):
    raw = text.encode()
    b += struct.pack("<Q", len(raw)) + raw


def _kv(b: bytearray, key: str, vtype: int, value):
    _s(b, key)
    b += struct.pack("<I", vtype)
    if vtype == T_UINT32:
        b += struct.pack("<I", value)
    elif vtype == T_INT32:
        b += struct.pack("<i", value)
    elif vtype == T_FLOAT32:
        b += struct.pack("<f", value)
    elif vtype == T_BOOL:
        b += struct.pack("<B", 1 if value else 0)
    elif vtype == T_STRING:
        _s(b, value)
    elif vtype == T_ARRAY:
        etype, items = value
        b += struct.pack("<IQ", etype, len(items))
        for it in items:
            if etype == T_STRING:
                _s(b, it)
            elif etype == T_FLOAT32:
                b += struct.pack("<f", it)
            elif etype == T_INT32:
                b += struct.pack("<i", it)
            else:
                raise ValueError(etype)
    else:
        raise ValueError(vtype)


def llama_metadata(cfg, vocab: int, eos: int = 2, bos: int = 1, freq_base: float | None = None) -> list:
    md = [
        ("general.architecture", T_STRING, "llama"),
        ("llama.context_length", T_UINT32, cfg.ctx_len),
        ("llama.embedding_length", T_UINT32, cfg.dim),
        ("llama.feed_forward_length", T_UINT32, cfg.ffn),
        ("llama.block_count", T_UINT32, cfg.n_layers),
        ("llama.attention.head_count", T_UINT32, cfg.n_heads),
        ("llama.attention.head_count_kv", T_UINT32, cfg.n_kv_heads),
        ("llama.rope.dimension_count", T_UINT32, cfg.dim // cfg.n_heads),
        ("llama.attention.layer_norm_rms_epsilon", T_FLOAT32, cfg.eps),
        ("tokenizer.ggml.tokens", T_ARRAY, (T_STRING, [f"<t{i}>" for i in range(vocab)])),
        ("tokenizer.ggml.scores", T_ARRAY, (T_FLOAT32, [0.0] * vocab)),
        ("tokenizer.ggml.token_type", T_ARRAY, (T_INT32, [1] * vocab)),
        ("tokenizer.ggml.bos_token_id", T_UINT32, bos),
        ("tokenizer.ggml.eos_token_id", T_UINT32, eos),
        ("tokenizer.ggml.unknown_token_id", T_UINT32, 0),
    ]
    if freq_base is not None:
        md.append(("llama.rope.freq_base", T_FLOAT32, freq_base))
    return md


def write_gguf(path: str, metadata: list, tensors: dict, alignment: int = 32, version: int = 3,
               magic: int = 0x46554747):
    """tensors: name -> numpy array (float16 -> GGML F16, float32 -> GGML F32), 1-D or 2-D, or an
    object with .blocks (uint8, the packed GGML blocks), .rows, .cols and .ggml_type (8 = Q8_0 if absent)."""
    head = bytearray()
    head += struct.pack("<IIQQ", magic, version, len(tensors), len(metadata))
    for key, vtype, value in metadata:
        _kv(head, key, vtype, value)
    offs, blobs, cur = [], [], 0
    for name, arr in tensors.items():
        _s(head, name)
        if hasattr(arr, "blocks"):
            head += struct.pack("<I", 2) + struct.pack("<QQ", arr.cols, arr.rows)
            ttype, raw = getattr(arr, "ggml_type", 8), np.ascontiguousarray(arr.blocks, np.uint8).tobytes()
        else:
            arr = np.ascontiguousarray(arr)
            ttype = 0 if arr.dtype == np.float32 else 1
            if arr.ndim == 1:
                head += struct.pack("<I", 1) + struct.pack("<Q", arr.shape[0])
            else:
                head += struct.pack("<I", 2) + struct.pack("<QQ", arr.shape[1], arr.shape[0])
            raw = arr.tobytes()
        head += struct.pack("<I", ttype) + struct.pack("<Q", cur)
        offs.append(cur)
        blobs.append(raw)
        cur += len(raw)
        cur = (cur + alignment - 1) // alignment * alignment
    data_start = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (data_start - len(head)))
        for off, raw in zip(offs, blobs):
            f.seek(data_start + off)
            f.write(raw)
        end = data_start + cur
        f.truncate(end)


def llama_tensors(cfg, weights: dict) -> dict:
    """GGUF tensors from f16 weights: norms as F32 1-D (the reference loader requires F32 norms)."""
    out = {}
    for name, w in weights.items():
        if name.endswith("norm.weight"):
            out[name] = np.ascontiguousarray(w.reshape(-1).astype(np.float32))
        else:
            out[name] = np.ascontiguousarray(w, dtype=np.float16)
    return out
