"""CPU-side checks of the C-ABI library: it loads, exports every declared symbol, keeps torch out
of its signatures, and its host-only logic (stop policy, GGUF contract) behaves as the reference."""
import os
import re

import numpy as np
import pytest

from conftest import REPO

HEADER = os.path.join(REPO, "include", "aesir_hip.h")


@pytest.fixture(scope="module")
def A():
    import aesir_hip

    return aesir_hip


def test_library_exports_every_declared_symbol(A):
    names = A.declared_functions()
    assert len(names) >= 40
    assert A.missing_exports() == []
    assert A.abi_version() == 1


def test_header_is_plain_c():
    raw = open(HEADER).read()
    assert 'extern "C"' in raw
    text = re.sub(r"/\*.*?\*/", "", raw, flags=re.S)
    for bad in ("torch", "at::", "std::", "template", "hipStream_t", "class "):
        assert bad not in text, bad


def test_every_entry_point_cites_the_reference_or_says_why_not():
    text = open(HEADER).read()
    # each declaration block is preceded by a comment; most cite a reference file:line
    assert len(re.findall(r"\.mojo:\d+", text)) >= 25


def test_stop_policy(A):
    """tests/test_inference.mojo:297-315 (generation_stop_reason, aesir.mojo:195-212)."""
    assert A.generation_stop_reason(2, 2, 1, 32, [], 8, 128) == "eos"
    assert A.generation_stop_reason(99, 2, 1, 32, [99], 8, 128) == "stop_token"
    assert A.generation_stop_reason(265, 2, 32, 32, [], 39, 128) == "length"
    assert A.generation_stop_reason(265, 2, 1, 32, [], 128, 128) == "context_exhausted"
    assert A.generation_stop_reason(265, 2, 1, 32, [], 8, 128) == ""


def test_stop_policy_matches_oracle(A, oracle):
    rng = np.random.default_rng(3)
    for _ in range(500):
        tok, eos, gen, mx, nxt, ctxl = (int(v) for v in rng.integers(0, 6, 6))
        stops = [int(v) for v in rng.integers(0, 6, int(rng.integers(0, 3)))]
        assert A.generation_stop_reason(tok, eos, gen, mx, stops, nxt, ctxl) == \
            oracle.stop_reason(tok, eos, gen, mx, stops, nxt, ctxl)


# ---------------------------------------------------------------- GGUF contract (no GPU)

@pytest.fixture()
def tiny_gguf(tmp_path, oracle):
    from gguf_tools import llama_metadata, llama_tensors, write_gguf

    cfg = oracle.Config(dim=64, n_layers=2, n_heads=8, n_kv_heads=4, ffn=172, vocab=512, ctx_len=128)
    w = oracle.synthetic_weights(cfg, 5)

    def make(name="m.gguf", md=None, tensors=None, **kw):
        path = str(tmp_path / name)
        write_gguf(path, md if md is not None else llama_metadata(cfg, cfg.vocab),
                   tensors if tensors is not None else llama_tensors(cfg, w), **kw)
        return path

    return cfg, w, make


def test_gguf_inspect_valid(A, tiny_gguf):
    cfg, _, make = tiny_gguf
    c, fb = A.gguf_inspect(make())
    assert (c.dim, c.n_layers, c.n_heads, c.n_kv_heads, c.ffn, c.vocab, c.ctx_len) == (64, 2, 8, 4, 172, 512, 128)
    assert c.rope_theta == 10000.0 and fb == 10000.0 and c.eos_token_id == 2


def test_gguf_freq_base_recorded_not_applied(A, oracle, tiny_gguf):
    from gguf_tools import llama_metadata

    cfg, _, make = tiny_gguf
    c, fb = A.gguf_inspect(make(md=llama_metadata(cfg, cfg.vocab, freq_base=500000.0)))
    assert fb == 500000.0 and c.rope_theta == 10000.0


@pytest.mark.parametrize("mutation,message", [
    ("magic", "GGUF magic bytes are invalid"),
    ("version", "Only GGUF version 3 is supported"),
    ("arch", "GGUF architecture is not supported: mistral"),
    ("missing", "GGUF is missing required tensor: blk.1.ffn_down.weight"),
    ("shape", "GGUF required tensor has an invalid shape: blk.0.attn_k.weight"),
    ("type", "GGUF required tensor has an invalid type: output_norm.weight"),
    ("truncated", "GGUF is truncated"),
    ("heads", "GGUF query heads are not divisible by KV heads"),
    ("rope_dim", "GGUF RoPE dimension does not match attention head size"),
    ("alignment", "GGUF alignment must be a power of two up to 4096"),
    ("eos", "Tokenizer eos_token_id is out of bounds"),
    ("q8_1", "Real inference slice supports only F16 and F32 tensors"),
    ("f32_matrix", "GGUF required tensor has an invalid type: output.weight"),
    ("overflow", "GGUF tensor byte size overflows the file: token_embd.weight"),
    ("huge", "GGUF tensor byte size overflows the file: token_embd.weight"),
])
def test_gguf_contract_errors(A, tiny_gguf, mutation, message):
    """loader/gguf.mojo:405-628 error paths, with the reference's message text."""
    from gguf_tools import T_FLOAT32, T_STRING, T_UINT32, llama_metadata, llama_tensors, write_gguf

    cfg, w, make = tiny_gguf
    md = llama_metadata(cfg, cfg.vocab)
    tensors = llama_tensors(cfg, w)
    kw = {}
    if mutation == "magic":
        kw["magic"] = 0x12345678
    elif mutation == "version":
        kw["version"] = 2
    elif mutation == "arch":
        md[0] = ("general.architecture", T_STRING, "mistral")
    elif mutation == "missing":
        del tensors["blk.1.ffn_down.weight"]
    elif mutation == "shape":
        tensors["blk.0.attn_k.weight"] = tensors["blk.0.attn_k.weight"][:16]
    elif mutation == "type":
        tensors["output_norm.weight"] = tensors["output_norm.weight"].astype(np.float16)
    elif mutation == "heads":
        md[6] = ("llama.attention.head_count_kv", T_UINT32, 3)
    elif mutation == "rope_dim":
        md[7] = ("llama.rope.dimension_count", T_UINT32, 4)
    elif mutation == "alignment":
        md.append(("general.alignment", T_UINT32, 48))
    elif mutation == "eos":
        md[13] = ("tokenizer.ggml.eos_token_id", T_UINT32, 9999)
    if mutation == "f32_matrix":
        # a matrix in F32: matrices are F16 (or one of the block types), never F32
        tensors["output.weight"] = tensors["output.weight"].astype(np.float32)
    path = make(md=md, tensors=tensors, **kw)
    if mutation == "truncated":
        size = os.path.getsize(path)
        with open(path, "r+b") as f:
            f.truncate(size - 100)
    if mutation in ("q8_1", "overflow", "huge"):
        # q8_1: rewrite the type field of the first tensor to GGML Q8_1 (9), which neither loader
        # takes; overflow: dims whose element count wraps int64 (2^33 x 2^31); huge: dims whose
        # byte size fits int64 but exceeds the file (2^20 x 2^20)
        raw = bytearray(open(path, "rb").read())
        name = b"token_embd.weight"
        i = raw.index(name) + len(name)
        ndim = int.from_bytes(raw[i:i + 4], "little")
        tpos = i + 4 + 8 * ndim
        if mutation == "q8_1":
            raw[tpos:tpos + 4] = (9).to_bytes(4, "little")
        else:
            ne0, ne1 = (1 << 33, 1 << 31) if mutation == "overflow" else (1 << 20, 1 << 20)
            raw[i + 4:i + 12] = ne0.to_bytes(8, "little")
            raw[i + 12:i + 20] = ne1.to_bytes(8, "little")
        open(path, "wb").write(bytes(raw))
    with pytest.raises(A.AesirError, match=re.escape(message)):
        A.gguf_inspect(path)


def test_gguf_duplicate_key(A, tiny_gguf):
    from gguf_tools import T_UINT32, llama_metadata

    cfg, _, make = tiny_gguf
    md = llama_metadata(cfg, cfg.vocab) + [("llama.block_count", T_UINT32, 2)]
    with pytest.raises(A.AesirError, match="duplicate metadata key: llama.block_count"):
        A.gguf_inspect(make(md=md))


def test_gguf_missing_file(A, tmp_path):
    with pytest.raises(A.AesirError, match="Failed to open GGUF model"):
        A.gguf_inspect(str(tmp_path / "nope.gguf"))


def test_q8_0_tensor_pack_matches_oracle_dequantize(A, oracle):
    """Q8_0Tensor packs GGUF block_q8_0 bytes; its dequantize equals the oracle's
    dequantize_q8_0 (compute.mojo:343-353) bit for bit."""
    rng = np.random.default_rng(3)
    q = rng.integers(-127, 128, size=(6, 96), dtype=np.int8)
    d = rng.uniform(0.001, 0.02, (6, 3)).astype(np.float16)
    t = A.Q8_0Tensor.from_parts(d, q)
    assert t.blocks.shape == (18, 34)
    assert np.array_equal(t.blocks[4, :2].view(np.float16), d.reshape(-1)[4:5])
    assert np.array_equal(t.blocks[4, 2:].view(np.int8), q.reshape(-1, 32)[4])
    ref = oracle.dequantize_q8_0(t.blocks, 18).reshape(6, 96)
    assert np.array_equal(t.dequantize().view(np.uint16), ref.view(np.uint16))


def test_gguf_inspect_q8_0_file(A, oracle, tmp_path):
    """A file whose matrices are all Q8_0 (norms F32) passes the loader contract."""
    from gguf_tools import llama_metadata, write_gguf

    cfg = oracle.Config(dim=64, n_layers=2, n_heads=4, n_kv_heads=2, ffn=96, vocab=128, ctx_len=64)
    tensors = {}
    for name, (r, c) in oracle.tensor_shapes(cfg).items():
        if name.endswith("norm.weight"):
            tensors[name] = np.ones(c, np.float32)
        else:
            tensors[name] = A.Q8_0Tensor.from_parts(np.full((r, c // 32), 0.01, np.float16), np.ones((r, c), np.int8))
    path = str(tmp_path / "q8.gguf")
    write_gguf(path, llama_metadata(cfg, cfg.vocab), tensors)
    c, _ = A.gguf_inspect(path)
    assert (c.dim, c.n_layers, c.ffn, c.vocab) == (64, 2, 96, 128)
    # a Q8_0 tensor whose rows are not whole blocks is rejected while mapping the tensor table
    from types import SimpleNamespace

    tensors["blk.0.ffn_down.weight"] = SimpleNamespace(blocks=np.zeros((160, 34), np.uint8), rows=64, cols=80)
    write_gguf(path, llama_metadata(cfg, cfg.vocab), tensors)
    with pytest.raises(A.AesirError, match="GGUF tensor row length is not a multiple of its block size: blk.0.ffn_down.weight"):
        A.gguf_inspect(path)


@pytest.mark.parametrize("kind", ["q4_0", "q4_k", "q6_k"])
def test_gguf_inspect_4bit_files(A, oracle, tmp_path, kind):
    """Files whose matrices are all Q4_0, Q4_K or Q6_K (norms F32) pass the loader contract, and so
    do files that mix block types between matrices; a matrix of a type outside the set (F32) is
    refused with the reference's type message."""
    from gguf_tools import llama_metadata, write_gguf

    cfg = oracle.Config(dim=256, n_layers=1, n_heads=4, n_kv_heads=2, ffn=512, vocab=64, ctx_len=32)
    rng = np.random.default_rng(1)

    def tensor(k, r, c):
        if k == "q4_0":
            return A.Q4_0Tensor.from_parts(np.full((r, c // 32), 0.01, np.float16), rng.integers(0, 16, (r, c)).astype(np.uint8))
        if k == "q4_k":
            n = c // 256
            return A.Q4_KTensor.from_parts(np.full((r, n), 0.001, np.float16), np.full((r, n), 0.001, np.float16),
                                           np.ones((r, n, 8), np.uint8), np.ones((r, n, 8), np.uint8),
                                           rng.integers(0, 16, (r, c)).astype(np.uint8))
        return A.Q6_KTensor.from_parts(np.full((r, c // 256), 0.001, np.float16), np.ones((r, c // 256, 16), np.int8),
                                       rng.integers(0, 64, (r, c)).astype(np.uint8))

    tensors = {}
    for name, (r, c) in oracle.tensor_shapes(cfg).items():
        tensors[name] = np.ones(c, np.float32) if name.endswith("norm.weight") else tensor(kind, r, c)
    path = str(tmp_path / "q.gguf")
    write_gguf(path, llama_metadata(cfg, cfg.vocab), tensors)
    c, _ = A.gguf_inspect(path)
    assert (c.dim, c.ffn, c.vocab) == (256, 512, 64)
    other = "q6_k" if kind != "q6_k" else "q4_k"
    tensors["blk.0.attn_v.weight"] = tensor(other, cfg.kv_dim, cfg.dim)
    tensors["blk.0.ffn_down.weight"] = A.Q8_0Tensor.from_parts(np.full((cfg.dim, cfg.ffn // 32), 0.01, np.float16),
                                                               np.ones((cfg.dim, cfg.ffn), np.int8))
    tensors["output.weight"] = np.zeros((cfg.vocab, cfg.dim), np.float16)
    write_gguf(path, llama_metadata(cfg, cfg.vocab), tensors)
    c, _ = A.gguf_inspect(path)
    assert (c.dim, c.ffn, c.vocab) == (256, 512, 64)
    tensors["blk.0.attn_v.weight"] = np.zeros((cfg.kv_dim, cfg.dim), np.float32)
    write_gguf(path, llama_metadata(cfg, cfg.vocab), tensors)
    with pytest.raises(A.AesirError, match="GGUF required tensor has an invalid type: blk.0.attn_v.weight"):
        A.gguf_inspect(path)
