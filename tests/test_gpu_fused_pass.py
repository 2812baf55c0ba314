"""The Q4_1 ring GEMM and the M <= 2 pipelined GEMV with Linear's gated
combine fused into the write-back (nnops_hip_gemm_q4_1_fused) against the two-step form it replaces
(nnops_hip_gemm_q4_1 into an f32 staging buffer, then
nnops_hip_fp_output_pass): the same products and the same pass arithmetic, so
the destinations must agree bit for bit. Covers gate activations, limit,
gate_beta, residual and an outer activation, f16 and f32 destinations, ragged
M and N; the plain pass (bias / activation / residual, MatMul's alpha / beta)
must be declined with the destination untouched. The two-step form itself is
checked against the oracle in test_gpu_linear_gated.py."""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import pytest

import datagen as dg
import nnops_amd as na
from gpu_util import dev, host, announce
from nnops_amd._lib import FpOutArgs

pytestmark = pytest.mark.gpu

VARIANTS = [
    dict(gated=1, gate_act=na.ACT_SILU, gate_alpha=1.0),
    dict(gated=1, gate_act=na.ACT_GELU, gate_beta=1.0, gate_limit=7.0, add_to=1),
    dict(gated=1, gate_act=na.ACT_SIGMOID, act=na.ACT_RELU),
    dict(act=na.ACT_GELU),
    dict(act=na.ACT_RELU, add_to=1, residual_pre=1),
    dict(act=na.ACT_TANH, add_to=1, min_clip=-0.5, max_clip=0.75),
    dict(matmul_order=1, alpha=0.5, beta=0.25),
    dict(matmul_order=1, alpha=1.0, beta=1.0, bias=False),
]


def _args(kw, M, n, out, bias, f16):
    fo = FpOutArgs()
    fo.out, fo.ld_out, fo.rows, fo.n = out.data_ptr(), out.stride(0), M, n
    fo.out_f16 = int(f16)
    fo.bias = bias.data_ptr() if bias is not None else None
    fo.min_clip, fo.max_clip = -math.inf, math.inf
    fo.gate_alpha, fo.gate_beta, fo.gate_limit = 1.0, 0.0, math.inf
    fo.alpha, fo.beta = 1.0, 0.0
    for k, v in kw.items():
        if k != "bias":
            setattr(fo, k, v)
    return fo


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("M,K,N", [(70, 512, 520), (200, 256, 1000), (1, 4096, 1001), (2, 4096, 520)])
@pytest.mark.parametrize("vi", range(len(VARIANTS)))
def test_fused_pass_matches_two_step(f16, M, K, N, vi):
    import torch
    kw = VARIANTS[vi]
    announce(f"fused pass {kw} M={M} K={K} N={N} f16={f16}")
    gated = bool(kw.get("gated"))
    n_w = 2 * N if gated else N
    tdt = torch.float16 if f16 else torch.float32
    a = dev(dg.normal(11 + vi, (M, K)).astype(np.float16))
    blk = dev(dg.q4_1_blocks(12 + vi, n_w, K))
    bias = None if kw.get("bias") is False else dev(dg.normal(13 + vi, (n_w,)).astype(np.float16 if f16 else np.float32))
    old = dg.normal(14 + vi, (M, N)).astype(np.float16 if f16 else np.float32)
    lib = na.lib()
    g = na.GemmQ41Args()
    g.a, g.b = a.data_ptr(), blk.data_ptr()
    g.m, g.n, g.k = M, n_w, K
    g.lda, g.ldb_bytes = K, blk.stride(0)
    g.trans_b, g.a_f16, g.out_kind = 1, 1, na.OUT_F32
    # two-step: f32 staging, then the pass
    stage = torch.empty((M, n_w), dtype=torch.float32, device="cuda")
    g.c, g.ldc = stage.data_ptr(), n_w
    need = lib.nnops_hip_gemm_q4_1_workspace_size(C.byref(g))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    y2 = dev(old.copy())
    assert lib.nnops_hip_gemm_q4_1(C.byref(g), ws.data_ptr(), need, None) == na.OK
    fo = _args(kw, M, N, y2, bias, f16)
    fo.src, fo.ld_src = stage.data_ptr(), n_w
    assert lib.nnops_hip_fp_output_pass(C.byref(fo), None) == na.OK
    # fused: the gated form; the plain pass is declined (nothing launched)
    y1 = dev(old.copy())
    g.c, g.ldc = None, 0
    fo1 = _args(kw, M, N, y1, bias, f16)
    rc = lib.nnops_hip_gemm_q4_1_fused(C.byref(g), C.byref(fo1), None)
    if not gated:
        assert rc == na.UNSUPPORTED, rc
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(y1), old)
        return
    assert rc == na.OK, rc
    torch.cuda.synchronize()
    got, want = host(y1), host(y2)
    assert got.dtype == (np.float16 if f16 else np.float32) and got.shape == (M, N)
    np.testing.assert_array_equal(got.view(np.uint16 if f16 else np.uint32),
                                  want.view(np.uint16 if f16 else np.uint32))
