"""Calls captured into a HIP graph and replayed (as bench.py times them):
every replay, with eager work and synchronizations between replays, must
reproduce the eager result bit for bit -- the routes with split-K partials
and a reduce, the fused ring passes, the GEMVs and the Q4_1 kernels."""
from __future__ import annotations

import numpy as np
import pytest

import datagen as dg
import nnops_amd as na
from gpu_util import dev, host, announce

pytestmark = pytest.mark.gpu


def graph_replays_match(fn, out, replays=3):
    import torch
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        fn(s)
    torch.cuda.synchronize()
    want = host(out).copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        fn(s)
    for r in range(replays):
        out.zero_()                       # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = host(out)
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), f"replay {r} differs"


@pytest.mark.parametrize("M,K,N,out,trans_b", [(4096, 1024, 1024, "s8", True), (333, 14336, 1024, "s8", True),
                                               (1024, 512, 1024, "f16", True), (16, 4096, 1024, "s32", True),
                                               (1, 4096, 2048, "s32", True), (1, 4096, 11008, "s8", False),
                                               (2, 4096, 2048, "s32", False), (16, 4096, 2048, "s8", False),
                                               (64, 1000, 1040, "s8", False)])
def test_int8_routes_under_graph_replay(M, K, N, out, trans_b):
    """[K,N] rows (trans_b False): the column GEMV and its split reduce for
    M <= 16, the tiled transpose into the workspace and the GEMM beyond."""
    import torch
    announce(f"graph int8 {M}x{K}x{N} {out} trans_b={trans_b}")
    a = dev(dg.act_s8(M + K, (M, K)))
    w = dev(dg.ints(N + 1, (N, K) if trans_b else (K, N), -127, 127))
    sb = dev(dg.uniform(3, (N,), 0.001, 0.01))
    tdt = {"s8": torch.int8, "f16": torch.float16, "s32": torch.int32}[out]
    c = torch.zeros((M, N), dtype=tdt, device="cuda")
    kind = {"s8": na.OUT_S8, "f16": na.OUT_F16, "s32": na.OUT_S32}[out]
    ws = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")

    def fn(s):
        na.gemm_i8(a, w, c, trans_b=trans_b, out_kind=kind, s_a=0.02, s_b=sb, s_out=0.05,
                   act=na.ACT_RELU if out != "s32" else na.ACT_NONE, workspace=ws, stream=s.cuda_stream)
    graph_replays_match(fn, c)


@pytest.mark.parametrize("trans_b", [True, False])
@pytest.mark.parametrize("a_dt", ["f16", "f32"])
def test_q4_1_under_graph_replay(trans_b, a_dt):
    """Both Q4_1 layouts; blocks along N at M <= 2 is the one-launch GEMV whose
    arrival counters carry the launch epoch baked into the graph; M=8 with
    blocks along K is the matrix-core GEMV; f32 activations at M=256 are
    split into two f16 parts in the workspace before the ring."""
    import torch
    announce(f"graph q4_1 trans_b={trans_b} a={a_dt}")
    K, N = 4096, 2048
    blk = dev(dg.q4_1_blocks(5, N, K) if trans_b else dg.q4_1_blocks(5, K, N))
    for M in (1, 2, 8, 256):
        a = dev(dg.normal(6 + M, (M, K)).astype(np.float16 if a_dt == "f16" else np.float32))
        c = torch.zeros((M, N), dtype=torch.float32, device="cuda")
        ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")

        def fn(s, a=a, c=c, ws=ws):
            na.gemm_q4_1(a, blk, c, n=N, trans_b=trans_b, workspace=ws, stream=s.cuda_stream)
        graph_replays_match(fn, c)


def test_quantize_linear_under_graph_replay():
    import torch
    announce("graph qdq")
    x = dev(dg.normal(7, (512, 1024)).astype(np.float16))
    sc = dev(dg.uniform(8, (512,), 0.01, 0.05))
    zp = dev(dg.ints(9, (512,), -4, 4, np.int8))
    q = torch.zeros((512, 1024), dtype=torch.int8, device="cuda")
    op = na.QuantizeLinear(axis=-1)
    ins = [na.tensor(x), na.tensor(sc), na.tensor(zp)]
    outs = [na.tensor(q)]

    def fn(s):
        assert op.compute(outs, ins, stream=s) == na.OK
    graph_replays_match(fn, q)


@pytest.mark.parametrize("M,K,N,trans_b", [(1, 4096, 2048, False), (4, 4096, 2048, True), (512, 4096, 1024, True),
                                           (1024, 256, 2048, False), (300, 1000, 200, True)])
def test_dense_fp_under_graph_replay(M, K, N, trans_b):
    """The dense f16 product: the [K,N] GEMV's split partials and their sum,
    the ring's split partials and reduce, the ring over a B transposed into
    the workspace, and the f32-MFMA tile kernel."""
    import torch
    announce(f"graph dense f16 {M}x{K}x{N} trans_b={trans_b}")
    a = dev(dg.normal(11 + M, (M, K)).astype(np.float16))
    b = dev(dg.normal(12, (N, K) if trans_b else (K, N)).astype(np.float16))
    c = torch.zeros((M, N), dtype=torch.float16, device="cuda")
    ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")

    def fn(s):
        na.gemm_fp(a, b, c, trans_b=trans_b, workspace=ws, stream=s.cuda_stream)
    graph_replays_match(fn, c)


def test_linear_gated_dense_under_graph_replay():
    """Linear's gated form over a dense f16 weight: the product staged in the
    workspace, then the output pass."""
    import torch
    announce("graph linear gated dense")
    M, K, N = 64, 1024, 512
    x = dev(dg.normal(13, (M, K)).astype(np.float16))
    w = dev((0.05 * dg.normal(14, (2 * N, K))).astype(np.float16))
    bias = dev((0.1 * dg.normal(15, (2 * N,))).astype(np.float16))
    y = torch.zeros((M, N), dtype=torch.float16, device="cuda")
    op = na.Linear(gated=True, gate_activation=na.EP_SILU)
    ins = [na.tensor(x), na.tensor(w), na.tensor(bias)]
    outs = [na.tensor(y)]
    ws = torch.empty(max(op.workspace_size(ins, outs), 1), dtype=torch.uint8, device="cuda")

    def fn(s):
        assert op.compute(outs, ins, stream=s, workspace=ws) == na.OK
    graph_replays_match(fn, y)
