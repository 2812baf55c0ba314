"""Helpers shared by the GPU parity tests."""
from __future__ import annotations

import sys

import numpy as np


def dev(x, device="cuda"):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(device)


def pitched(x, pitch_elems, device="cuda"):
    """Device copy of 2-D ``x`` inside a wider buffer (row pitch > width),
    padding filled with a sentinel so a read past the row shows up."""
    import torch
    rows, cols = x.shape
    buf = np.full((rows, pitch_elems), 0x5A if x.dtype.itemsize == 1 else 7, dtype=x.dtype)
    buf[:, :cols] = x
    t = torch.from_numpy(buf).to(device)
    return t[:, :cols]


def host(t):
    return t.detach().cpu().numpy()


def announce(msg):
    """Name the case before a GPU step, flushed, so a fault can be traced."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def q41_f16_weights(M, K, f16, trans_b=True, N=None, packed=False):
    """Whether the Q4_1 route for M x K decodes its weights to f16 (the oracle's
    w_round_f16): f16 A past M = 2, and f32 A on the split-f16 rings (K % 64
    == 0, past the GEMV rows M <= 16; blocks along K past the skinny rows M <=
    48 with K % 256 == 0; blocks along N with 16-byte weight rows, i.e. N a
    multiple of 128, or the prepacked planes)."""
    if f16:
        return M > 2
    if K % 64 or M <= 16:
        return False
    if trans_b:
        return not (M <= 48 and K % 256 == 0)
    return packed or ((N + 31) // 32 * 20) % 16 == 0


def norm_err(got, want):
    """max |got - want| / max(|want|, rms(want)), elementwise: a relative error
    that stays meaningful at outputs that cancel to ~0 (the tolerance metric of
    the Q4_1 routes)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rms = np.sqrt(np.mean(want * want)) if want.size else 1.0
    den = np.maximum(np.abs(want), rms)
    return float(np.max(np.abs(got - want) / den)) if want.size else 0.0


def oracle_rows(fn, m, band=16, threads=None):
    """Every row of an M-row oracle result, computed in row bands of `band`
    on a thread pool (the oracle's C calls release the GIL): fn(r0, r1)
    returns rows [r0, r1) of the result. Lets the full-size configurations
    be compared in full within seconds."""
    import concurrent.futures as cf
    import os
    if threads is None:
        threads = max(1, min(16, len(os.sched_getaffinity(0))))
    starts = list(range(0, m, band))
    with cf.ThreadPoolExecutor(threads) as ex:
        parts = list(ex.map(lambda r0: fn(r0, min(m, r0 + band)), starts))
    return np.concatenate(parts, axis=0)
