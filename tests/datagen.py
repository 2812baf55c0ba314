"""Seeded synthetic inputs for the tests (and the golden-fixture generator).

Values come from the xorshift128+ stream of nnops' test harness
(tests/common/random_tensor.hpp:18-57), exposed by the oracle library as
orc_xs128_u64, so a (seed, shape) pair names the same bytes everywhere.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

import oracle


def u64(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint64)
    lib = oracle.lib()
    lib.orc_xs128_u64.argtypes = [C.c_uint64, C.c_int64, C.c_void_p]
    lib.orc_xs128_u64(seed, count, out.ctypes.data)
    return out


def unit(seed: int, count: int) -> np.ndarray:
    """Floats in [0, 1) from the low 24 bits (the harness's next_float)."""
    return (u64(seed, count) & np.uint64(0xFFFFFF)).astype(np.float32) / np.float32(16777216.0)


def ints(seed: int, shape, lo: int, hi: int, dtype=np.int8) -> np.ndarray:
    """Uniform integers in [lo, hi] (inclusive)."""
    n = int(np.prod(shape))
    span = np.uint64(hi - lo + 1)
    v = (u64(seed, n) % span).astype(np.int64) + lo
    return v.astype(dtype).reshape(shape)


def uniform(seed: int, shape, lo: float, hi: float) -> np.ndarray:
    n = int(np.prod(shape))
    return (np.float32(lo) + unit(seed, n) * np.float32(hi - lo)).astype(np.float32).reshape(shape)


def normal(seed: int, shape, sigma: float = 1.0) -> np.ndarray:
    """Box-Muller over the seeded stream (float64 math, float32 result)."""
    n = int(np.prod(shape))
    m = (n + 1) // 2
    u = u64(seed, 2 * m)
    u1 = ((u[:m] >> np.uint64(11)).astype(np.float64) + 0.5) / 9007199254740992.0
    u2 = (u[m:] >> np.uint64(11)).astype(np.float64) / 9007199254740992.0
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])[:n]
    return (z * sigma).astype(np.float32).reshape(shape)


def act_s8(seed: int, shape, sigma: float = 30.0) -> np.ndarray:
    """Activations round(N(0, sigma)) clipped to [-127, 127]."""
    return np.clip(np.rint(normal(seed, shape, sigma)), -127, 127).astype(np.int8)


def q4_1_blocks(seed: int, rows: int, cols: int) -> np.ndarray:
    """rows x ceil(cols/32) Q4_1 blocks with d ~ U(0.001, 0.02) and
    m ~ U(-0.1, 0) rounded to f16, nibbles uniform 0..15.
    Returns uint8 [rows, nb*20]."""
    nb = (cols + 31) // 32
    d = uniform(seed, (rows, nb), 0.001, 0.02).astype(np.float16)
    mn = uniform(seed + 1, (rows, nb), -0.1, 0.0).astype(np.float16)
    qs = ints(seed + 2, (rows, nb, 16), 0, 255, np.uint8)
    blk = np.zeros((rows, nb, 20), dtype=np.uint8)
    blk[:, :, 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:4] = mn.view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 4:] = qs
    return blk.reshape(rows, nb * 20)
