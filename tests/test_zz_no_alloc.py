"""nnops_hip_gemm_i8_noalloc (the library's fixed device scratch in place of a
caller workspace) against nnops_hip_gemm_i8 with a caller workspace, bit for
bit, on two calls in a row (the second smaller, so it runs over what the
first left in the scratch), plus the limit's rejection."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import datagen as dg
import nnops_amd as na
from gpu_util import dev, host, pitched, announce

pytestmark = pytest.mark.gpu

LIMIT = 64 << 20


def _pair(a, b, c0, **kw):
    import torch
    ref = c0.clone()
    na.gemm_i8(a, b, ref, **kw)
    got = c0.clone()
    na.gemm_i8(a, b, got, noalloc=True, **kw)
    torch.cuda.synchronize()
    return host(got), host(ref)


def _need(M, N, K, trans_b, **fields):
    g = na.GemmI8Args()
    g.m, g.n, g.k, g.trans_b = M, N, K, int(trans_b)
    for k, v in fields.items():
        setattr(g, k, v)
    return na.lib().nnops_hip_gemm_i8_workspace_size(C.byref(g))


def test_noalloc_first_call_under_graph_capture():
    """The entry point's first call in the process is made while a stream is
    captured (its one-time scratch lookup then runs inside the capture): the
    K-split plan (int32 partials in the scratch, then the reduce with the
    float epilogue and add_to) replayed three times, C restored eagerly
    between replays, each replay equal bit for bit to the workspace route."""
    import torch
    M, K, N = 333, 14336, 1024
    assert _need(M, N, K, True, out_kind=na.OUT_S8, float_ep=1, add_to=1, act=na.ACT_GELU) > (1 << 20)
    announce("noalloc under graph capture: 333x14336x1024 float epilogue, K split")
    a = pitched(dg.act_s8(531, (M, K)), 14400)
    w = dev(dg.ints(532, (N, K), -127, 127))
    sb = dev(dg.uniform(533, (N,), 0.001, 0.01))
    bias = dev(dg.ints(534, (N,), -5000, 5000, np.int32))
    c0 = pitched(dg.ints(535, (M, N), -128, 127), 1040)
    kw = dict(trans_b=True, bias=bias, out_kind=na.OUT_S8, s_a=0.02, s_b=sb, s_out=2.0, float_ep=True,
              act=na.ACT_GELU, add_to=True)
    want = c0.clone()
    na.gemm_i8(a, w, want, **kw)
    torch.cuda.synchronize()
    want = host(want)
    c = c0.clone()
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        na.gemm_i8(a, w, c, noalloc=True, stream=s.cuda_stream, **kw)
    for r in range(3):
        c.copy_(c0)                       # eager work between replays: the residual restored
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(c), want, err_msg=f"replay {r}")
    assert np.unique(want).size > 50


def test_noalloc_matches_workspace_route_two_calls():
    import torch
    # 1: config 5's Linear form (K split 4 ways: ~21.8 MB of int32 partials in
    #    the scratch), s8 add_to + GELU on pitched A and C
    M, K, N = 333, 14336, 4096
    assert 16 << 20 < _need(M, N, K, True, out_kind=na.OUT_S8, float_ep=1, add_to=1, act=na.ACT_GELU) <= LIMIT
    announce("noalloc call 1: 333x14336x4096 float epilogue, K-split partials in the scratch")
    a = pitched(dg.act_s8(501, (M, K)), 14400)
    w = dev(dg.ints(502, (N, K), -127, 127))
    sb = dev(dg.uniform(503, (N,), 0.001, 0.01))
    bias = dev(dg.ints(504, (N,), -5000, 5000, np.int32))
    c0 = pitched(dg.ints(505, (M, N), -128, 127), 4160)
    got, want = _pair(a, w, c0, trans_b=True, bias=bias, out_kind=na.OUT_S8, s_a=0.02, s_b=sb, s_out=2.0,
                      float_ep=True, act=na.ACT_GELU, add_to=True)
    np.testing.assert_array_equal(got, want)
    assert np.unique(want).size > 50
    # 2: smaller, another plan over the same scratch: a [K,N] B staged
    #    transposed, zero points (row / column sums), u8 A, requant
    M, K, N = 40, 1024, 520
    assert 0 < _need(M, N, K, False, zp_a_scalar=3) < _need(333, 4096, 14336, True, out_kind=na.OUT_S8,
                                                            float_ep=1, add_to=1)
    announce("noalloc call 2: 40x1024x520 [K,N] u8 A with zero points")
    a = dev(dg.ints(511, (M, K), 0, 255, np.uint8))
    b = dev(dg.ints(512, (K, N), -127, 127))
    c0 = torch.zeros((M, N), dtype=torch.int8, device="cuda")
    got, want = _pair(a, b, c0, trans_b=False, out_kind=na.OUT_S8, s_a=0.03, zp_a=128, zp_b=2, s_b=0.01,
                      s_out=1.5, zp_out=-3)
    np.testing.assert_array_equal(got, want)
    # 3: a GEMV over a [K,N] weight (its K-split partials in the scratch)
    announce("noalloc call 3: M=1 [K,N] GEMV")
    M, K, N = 1, 4096, 11008
    a = dev(dg.ints(521, (M, K), -127, 127))
    b = dev(dg.ints(522, (K, N), -127, 127))
    c0 = torch.zeros((M, N), dtype=torch.int32, device="cuda")
    got, want = _pair(a, b, c0, trans_b=False)
    np.testing.assert_array_equal(got, want)


def test_noalloc_rejects_a_plan_beyond_the_scratch():
    # a raw [K,N] weight at config 5's shape with an A zero point (the
    # compensation needs B's column sums, so B is staged transposed: 58.7 MB)
    # beside the partials: more than the scratch holds, rejected before any launch
    import torch
    M, K, N = 333, 14336, 4096
    assert _need(M, N, K, False, out_kind=na.OUT_S8, float_ep=1, add_to=1, zp_a_scalar=3) > LIMIT
    announce("noalloc rejection")
    a = torch.zeros((M, K), dtype=torch.int8, device="cuda")
    b = torch.zeros((K, N), dtype=torch.int8, device="cuda")
    c = torch.full((M, N), 7, dtype=torch.int8, device="cuda")
    rc = na.gemm_i8(a, b, c, trans_b=False, out_kind=na.OUT_S8, float_ep=True, add_to=True, zp_a=3,
                    noalloc=True, check=False)
    torch.cuda.synchronize()
    assert rc == na.OUT_OF_MEMORY
    assert bool((c == 7).all())
