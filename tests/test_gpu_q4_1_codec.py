"""The device Q4_1 codec (nnops_hip_q4_1_quantize / _dequantize) against the
reference's quantize_q4 / pack_q4: byte-identical blocks on the golden
fixtures written by the reference's compiled quantize_q4 (tests/golden), on
partial blocks, and against the oracle (itself pinned to the reference) on
rows with a pitch; the decode bit-identical to the oracle's."""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import pytest

import oracle
import datagen as dg
import nnops_amd as na
from gpu_util import dev, host, announce

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden.json")))


@pytest.mark.parametrize("entry", GOLD["q4_1_quantize"], ids=lambda e: str(e["count"]))
def test_quantize_golden_bytes(entry):
    announce(f"q4_1 quantize golden count={entry['count']}")
    import torch
    x = dg.uniform(entry["seed"], (1, entry["count"]), -1.0, 1.0)
    got = host(na.q4_1_quantize(dev(x)))
    torch.cuda.synchronize()
    assert hashlib.sha256(got.tobytes()).hexdigest() == entry["out"]["sha256"]


@pytest.mark.parametrize("rows,cols,pitch,f16", [(3, 1, 8, False), (5, 33, 40, False), (7, 71, 96, True),
                                                 (64, 4096, 4096, False), (130, 1000, 1032, True),
                                                 (1024, 14336, 14336, True)])
def test_quantize_rows_match_oracle(rows, cols, pitch, f16):
    """Pitched rows, partial last blocks, f32 and f16 sources, equal-valued
    blocks (d = 0) and a weight-sized matrix."""
    announce(f"q4_1 quantize {rows}x{cols} pitch={pitch} f16={f16}")
    import torch
    x = dg.normal(rows * 31 + cols, (rows, pitch)).astype(np.float16 if f16 else np.float32)
    x[0, :min(cols, 40)] = 0.25          # constant blocks: d = 0
    if rows > 2:
        x[2, :cols] = np.linspace(-3, 5, cols)
    xd = dev(x)[:, :cols]
    got = host(na.q4_1_quantize(xd))
    want = np.stack([oracle.q4_1_quantize(np.ascontiguousarray(x[r, :cols], np.float32)) for r in range(rows)])
    np.testing.assert_array_equal(got, want)
    # and back: pack_q4 on the device equals the oracle's decode bit for bit
    back = host(na.q4_1_dequantize(dev(got), cols))
    ref = np.stack([oracle.q4_1_decode(want[r], cols) for r in range(rows)])
    np.testing.assert_array_equal(back.view(np.uint32), ref.view(np.uint32))
    back16 = host(na.q4_1_dequantize(dev(got), cols, dtype=torch.float16))
    np.testing.assert_array_equal(back16.view(np.uint16), ref.astype(np.float16).view(np.uint16))
