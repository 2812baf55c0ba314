"""GGUF container reading (host only): header, metadata (scalars, strings,
arrays), tensor descriptors, the aligned data section, and the Q4_1 / I8
weights read back byte for byte through the memory map."""
from __future__ import annotations

import struct

import numpy as np
import pytest

import datagen as dg
from nnops_amd import gguf


def test_roundtrip_q4_1_and_i8(tmp_path):
    N, K = 48, 320
    blocks = dg.q4_1_blocks(7, N, K)              # [N, K/32*20]
    w8 = dg.ints(8, (N, 96), -127, 127)
    p = str(tmp_path / "w.gguf")
    gguf.write_gguf(p, {"blk.0.ffn_up.weight": (gguf.GGML_Q4_1, (K, N), blocks.tobytes()),
                        "blk.0.attn_q.weight": (gguf.GGML_I8, (96, N), w8.tobytes())},
                    metadata={"general.architecture": "llama", "llama.block_count": 1})
    g = gguf.open_gguf(p)
    assert g.version == 3 and g.alignment == 32
    assert g.metadata["general.architecture"] == "llama" and g.metadata["llama.block_count"] == 1
    t = g.tensors["blk.0.ffn_up.weight"]
    assert t.dims == (K, N) and t.ggml_type == gguf.GGML_Q4_1 and t.offset % 32 == 0
    assert t.row_bytes == K // 32 * 20
    np.testing.assert_array_equal(g.raw("blk.0.ffn_up.weight"), blocks)
    np.testing.assert_array_equal(g.raw("blk.0.attn_q.weight").view(np.int8), w8)
    g.close()


def test_metadata_arrays_and_alignment(tmp_path):
    # a hand-built file: one u32 array kv, general.alignment = 64, one f32 tensor
    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    body = struct.pack("<IIQQ", gguf.GGUF_MAGIC, 3, 1, 2)
    body += s("general.alignment") + struct.pack("<II", 4, 64)
    body += s("tokenizer.ggml.token_type") + struct.pack("<IIQ", 9, 4, 3) + struct.pack("<3I", 1, 2, 3)
    body += s("x") + struct.pack("<I", 1) + struct.pack("<Q", 5) + struct.pack("<IQ", gguf.GGML_F32, 0)
    body += b"\0" * ((-len(body)) % 64)
    body += np.arange(5, dtype=np.float32).tobytes()
    p = tmp_path / "a.gguf"
    p.write_bytes(body)
    g = gguf.open_gguf(str(p))
    assert g.alignment == 64 and g.metadata["tokenizer.ggml.token_type"] == [1, 2, 3]
    assert g.tensors["x"].offset % 64 == 0
    np.testing.assert_array_equal(g.raw("x").view(np.float32).ravel(), np.arange(5, dtype=np.float32))
    g.close()


def test_rejects_non_gguf(tmp_path):
    p = tmp_path / "b.bin"
    p.write_bytes(b"NOPE" + b"\0" * 60)
    with pytest.raises(ValueError):
        gguf.open_gguf(str(p))
