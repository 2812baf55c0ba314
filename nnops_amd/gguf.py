"""GGUF weight files -> device weights for the Q4_1 / int8 routes.

A GGUF file (llama.cpp's container, version 2 and 3) is a header, metadata
key/values, tensor descriptors and an aligned data section. A Q4_1 tensor with
dims ne = [K, N] (ne[0] contiguous) is N rows of K/32 llama.cpp blocks -- f16
d, f16 m, 16 nibble bytes -- which is exactly the ``transpose_b`` (Linear,
[N, K]) form the Q4_1 kernels read in place (nnops' q4_1.hpp:5-18 block
layout; its decode takes an unaligned slice of such a file by memcpy). This
module reads the layout with a memory map (no copy on the host), and uploads
one tensor into device memory with the 16-byte base alignment the kernels
want; an s8 (GGML I8) tensor loads the same way as an int8 weight.

Only the container is parsed; nothing in the file is executed.
"""
from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass, field

import numpy as np

GGUF_MAGIC = 0x46554747  # "GGUF" little-endian

# ggml_type values used here (ggml.h): the block sizes of the types this path reads
GGML_F32, GGML_F16, GGML_Q4_1, GGML_I8 = 0, 1, 3, 24
_TYPE_BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_Q4_1: (32, 20), GGML_I8: (1, 1)}

# metadata value types (gguf.h)
_U8, _I8, _U16, _I16, _U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _I64, _F64 = range(13)
_SCALAR = {_U8: "<B", _I8: "<b", _U16: "<H", _I16: "<h", _U32: "<I", _I32: "<i", _F32: "<f",
           _BOOL: "<?", _U64: "<Q", _I64: "<q", _F64: "<d"}


@dataclass
class TensorInfo:
    name: str
    dims: tuple          # ne[0] first (the contiguous dimension)
    ggml_type: int
    offset: int          # absolute byte offset in the file

    @property
    def rows(self) -> int:
        return int(np.prod(self.dims[1:])) if len(self.dims) > 1 else 1

    @property
    def row_bytes(self) -> int:
        per, nbytes = _TYPE_BLOCK[self.ggml_type]
        return (self.dims[0] + per - 1) // per * nbytes

    @property
    def nbytes(self) -> int:
        return self.rows * self.row_bytes


@dataclass
class GGUFFile:
    path: str
    version: int
    metadata: dict = field(default_factory=dict)
    tensors: dict = field(default_factory=dict)
    alignment: int = 32
    _mm: mmap.mmap | None = None

    def raw(self, name: str) -> np.ndarray:
        """The tensor's bytes as a uint8 [rows, row_bytes] view of the map."""
        t = self.tensors[name]
        if t.ggml_type not in _TYPE_BLOCK:
            raise ValueError(f"{name}: ggml type {t.ggml_type} is not read by this path")
        buf = np.frombuffer(self._mm, dtype=np.uint8, count=t.nbytes, offset=t.offset)
        return buf.reshape(t.rows, t.row_bytes)

    def close(self):
        if self._mm is not None:
            self._mm.close()
            self._mm = None


class _Reader:
    def __init__(self, mm):
        self.mm = mm
        self.pos = 0

    def take(self, fmt):
        v = struct.unpack_from(fmt, self.mm, self.pos)[0]
        self.pos += struct.calcsize(fmt)
        return v

    def string(self):
        n = self.take("<Q")
        s = bytes(self.mm[self.pos:self.pos + n]).decode("utf-8")
        self.pos += n
        return s

    def value(self, vt):
        if vt in _SCALAR:
            return self.take(_SCALAR[vt])
        if vt == _STR:
            return self.string()
        if vt == _ARR:
            et = self.take("<I")
            n = self.take("<Q")
            return [self.value(et) for _ in range(n)]
        raise ValueError(f"unknown GGUF metadata type {vt}")


def open_gguf(path: str) -> GGUFFile:
    """Parse the header, metadata and tensor descriptors of a GGUF file."""
    f = open(path, "rb")
    try:
        mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    finally:
        f.close()
    r = _Reader(mm)
    if r.take("<I") != GGUF_MAGIC:
        mm.close()
        raise ValueError(f"{path}: not a GGUF file")
    version = r.take("<I")
    if version not in (2, 3):
        mm.close()
        raise ValueError(f"{path}: GGUF version {version} not supported")
    n_tensors = r.take("<Q")
    n_kv = r.take("<Q")
    g = GGUFFile(path=path, version=version, _mm=mm)
    for _ in range(n_kv):
        key = r.string()
        g.metadata[key] = r.value(r.take("<I"))
    g.alignment = int(g.metadata.get("general.alignment", 32))
    infos = []
    for _ in range(n_tensors):
        name = r.string()
        nd = r.take("<I")
        dims = tuple(r.take("<Q") for _ in range(nd))
        infos.append((name, dims, r.take("<I"), r.take("<Q")))
    data_start = (r.pos + g.alignment - 1) // g.alignment * g.alignment
    for name, dims, tt, off in infos:
        g.tensors[name] = TensorInfo(name, dims, tt, data_start + off)
    return g


def load_weight(g: GGUFFile, name: str, device="cuda"):
    """Upload one 2-D weight for Linear / MatMul(transpose_b=True).

    Returns ``(tensor, dtype_code, (N, K))``: a device uint8 [N, K/32*20]
    block buffer with ``DT_Q4_1`` for a Q4_1 tensor, an int8 [N, K] tensor
    with ``DT_S8`` for an I8 one. torch allocations are 256-byte aligned, so
    the kernels' aligned paths apply whatever the file offset was."""
    import torch
    from . import _lib as L
    t = g.tensors[name]
    if len(t.dims) != 2:
        raise ValueError(f"{name}: a {len(t.dims)}-D tensor is not a matmul weight")
    K, N = t.dims
    raw = g.raw(name)
    if t.ggml_type == GGML_Q4_1:
        return torch.from_numpy(np.array(raw)).to(device), L.DT_Q4_1, (N, K)
    if t.ggml_type == GGML_I8:
        return torch.from_numpy(np.array(raw).view(np.int8)).to(device), L.DT_S8, (N, K)
    raise ValueError(f"{name}: ggml type {t.ggml_type} has no quantized matmul route")


def write_gguf(path: str, tensors: dict, metadata: dict | None = None, alignment: int = 32):
    """Write a GGUF v3 file: ``tensors`` maps name -> (ggml_type, dims (ne[0]
    first), raw bytes). Used to build test fixtures; strings and integers
    only in ``metadata``."""
    md = dict(metadata or {})
    if alignment != 32:
        md["general.alignment"] = alignment

    def s(x):
        b = x.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    out = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(md)))
    for k, v in md.items():
        out += s(k)
        if isinstance(v, str):
            out += struct.pack("<I", _STR) + s(v)
        elif isinstance(v, float):
            out += struct.pack("<If", _F32, v)
        else:
            out += struct.pack("<IQ", _U64, v) if v >= 2 ** 32 else struct.pack("<II", _U32, v)
    offs, cur = [], 0
    for name, (tt, dims, data) in tensors.items():
        offs.append(cur)
        cur = (cur + len(data) + alignment - 1) // alignment * alignment
        out += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", tt, offs[-1])
    pad = (-len(out)) % alignment
    out += b"\0" * pad
    base = len(out)
    for (name, (tt, dims, data)), off in zip(tensors.items(), offs):
        out += b"\0" * (base + off - len(out))
        out += bytes(data)
    with open(path, "wb") as f:
        f.write(out)
