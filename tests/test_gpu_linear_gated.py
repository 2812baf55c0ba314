"""Linear's gated form (SwiGLU / GeGLU) and the fp epilogue (bias, residual,
activation) over Q4_1 weights, through the operator C facade on the GPU,
against the oracle: the f32 dequant GEMM (f64 accumulation) followed by
orc_fp_out_pass, which tests/test_oracle.py pins to nnops' own CPU Linear.

Bar: the Q4_1 tolerance (BASELINE: 2e-3) as a normalized error,
max_i |g_i - w_i| / max(|w_i|, rms(w)), for f32 and f16 destinations (an f16
rounding flip is 2^-10 of the value). Past M = 2 an f16 X takes the ring GEMM,
which decodes the weight to f16 as nnops' packed route does for half operands
(its small-M route decodes in f32), and so does an f32 X past the skinny
rows (the split-f16 ring); the oracle follows (w_round_f16, q41_f16_weights)."""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
import datagen as dg
import nnops_amd as na
from gpu_util import dev, host, announce, norm_err, oracle_rows, q41_f16_weights

pytestmark = pytest.mark.gpu

TOL = 2e-3


def run_linear(x, blk, n_w, *, gated, bias=None, old=None, f16_out=None, **attrs):
    """Linear over a q4_1 weight [n_w, K] (blocks along K); returns the output."""
    import torch
    M, K = x.shape
    f16 = x.dtype == np.float16 if f16_out is None else f16_out
    n = n_w // 2 if gated else n_w
    tdt = torch.float16 if f16 else torch.float32
    y = torch.zeros((M, n), dtype=tdt, device="cuda") if old is None else dev(old.astype(np.float16 if f16 else np.float32))
    op = na.Linear(gated=gated, **attrs)
    ins = [na.tensor(dev(x)), na.tensor(dev(blk), dtype=na.DT_Q4_1, shape=[n_w, K])]
    if bias is not None:
        ins.append(na.tensor(dev(bias)))
    outs = [na.tensor(y)]
    shape, dt = op.output_desc(ins)
    assert shape == [M, n]
    assert op.validate(ins, outs) == na.OK
    rc = op.compute(outs, ins)
    assert rc == na.OK, rc
    torch.cuda.synchronize()
    return host(y).astype(np.float32)


GATE = {na.EP_SILU: oracle.ACT_SILU, na.EP_GELU: oracle.ACT_GELU, na.EP_RELU: oracle.ACT_RELU,
        na.EP_SIGMOID: oracle.ACT_SIGMOID, na.EP_TANH: oracle.ACT_TANH, na.EP_NONE: oracle.ACT_NONE}


@pytest.mark.parametrize("M", [1, 512])
@pytest.mark.parametrize("gate", [na.EP_SILU, na.EP_GELU])
def test_gated_ffn_config4_shape(M, gate):
    """The decode / prefill FFN: f16 X [M, 4096] x q4_1 [2 x 14336, 4096]
    (gate rows, then value rows) with bias -> f16 [M, 14336]; every output
    checked, for M=1 (the GEMV route) and M=512 (the ring route)."""
    announce(f"gated ffn M={M} gate={gate}")
    K, N = 4096, 14336
    x = dg.normal(800 + M, (M, K)).astype(np.float16)
    blk = dg.q4_1_blocks(801, 2 * N, K)
    bias = (0.1 * dg.normal(802, (2 * N,))).astype(np.float16)
    got = run_linear(x, blk, 2 * N, gated=True, bias=bias, gate_activation=gate)
    want = oracle_rows(lambda r0, r1: oracle.q4_1_linear(x, blk, 2 * N, rows=(r0, r1), w_round_f16=M > 2, gated=True,
                                                         out_f16=True, bias=bias, gate_act=GATE[gate]), M,
                       band=4).astype(np.float32)
    err = norm_err(got, want)
    assert err <= TOL, err


@pytest.mark.parametrize("M,N", [(1, 1001), (2, 1001), (2, 512)])
@pytest.mark.parametrize("kw", [dict(gate_activation=na.EP_SILU), dict(gate_activation=na.EP_GELU, add_to=True)])
def test_gated_gemv_fused_edges(M, N, kw):
    """The one-launch gated GEMV (K = 4096, M <= 2, f16 X and destination)
    against the oracle: an odd output count (the last wave's column pair has
    one member), M = 2 (two rows per wave), the f16 pairs written as one
    word, and add_to (the destination read before the stream). Its f32
    destination is compared bit for bit with the two-step form in
    test_gpu_fused_pass.py."""
    announce(f"gated gemv M={M} N={N} {kw}")
    K = 4096
    f16 = True
    dt = np.float16
    x = dg.normal(900 + M, (M, K)).astype(np.float16)
    blk = dg.q4_1_blocks(901 + N, 2 * N, K)
    bias = (0.1 * dg.normal(902, (2 * N,))).astype(np.float16 if f16 else np.float32)
    old = dg.normal(903, (M, N)).astype(dt) if kw.get("add_to") else None
    got = run_linear(x, blk, 2 * N, gated=True, bias=bias, old=old, f16_out=f16, **kw)
    want = oracle.q4_1_linear(x, blk, 2 * N, w_round_f16=False, gated=True, out_f16=f16, bias=bias, out=old,
                              gate_act=GATE[kw["gate_activation"]],
                              add_to=kw.get("add_to", False)).astype(np.float32)
    err = norm_err(got, want)
    assert err <= TOL, err


GATED_VARIANTS = [
    dict(gate_activation=na.EP_SILU, gate_alpha=1.702, gate_beta=1.0, gate_limit=7.0),
    dict(gate_activation=na.EP_GELU, gate_beta=0.5, gate_limit=1.5, act=na.EP_RELU),
    dict(gate_activation=na.EP_SIGMOID, act=na.EP_TANH),
    dict(gate_activation=na.EP_TANH, add_to=True),
    dict(gate_activation=na.EP_RELU, min_clip=-0.3, max_clip=0.4, add_to=True),
    dict(gate_activation=na.EP_NONE),
]


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("M,K,N2", [(3, 256, 104), (70, 512, 520)])
@pytest.mark.parametrize("kw", GATED_VARIANTS)
def test_gated_variants(f16, M, K, N2, kw):
    announce(f"gated {M}x{K}x{N2} f16={f16} {kw}")
    dt = np.float16 if f16 else np.float32
    x = dg.normal(M + K, (M, K)).astype(dt)
    blk = dg.q4_1_blocks(N2, N2, K)
    bias = dg.normal(N2 + 1, (N2,)).astype(dt)
    old = dg.normal(N2 + 2, (M, N2 // 2)).astype(dt) if kw.get("add_to") else None
    got = run_linear(x, blk, N2, gated=True, bias=bias, old=old, **kw)
    want = oracle.q4_1_linear(x, blk, N2, w_round_f16=q41_f16_weights(M, K, f16), gated=True, out_f16=f16, bias=bias,
                              out=old,
                              gate_act=GATE[kw["gate_activation"]], gate_alpha=kw.get("gate_alpha", 1.0),
                              gate_beta=kw.get("gate_beta", 0.0), gate_limit=kw.get("gate_limit", math.inf),
                              act={None: oracle.ACT_NONE, na.EP_RELU: oracle.ACT_RELU,
                                   na.EP_TANH: oracle.ACT_TANH}[kw.get("act")],
                              min_clip=kw.get("min_clip", -math.inf), max_clip=kw.get("max_clip", math.inf),
                              add_to=kw.get("add_to", False)).astype(np.float32)
    err = norm_err(got, want)
    assert err <= TOL, err


PASS_VARIANTS = [
    dict(act=na.EP_GELU), dict(act=na.EP_SILU, add_to=True),
    dict(act=na.EP_RELU, min_clip=-0.5, max_clip=0.7, add_to=True, residual_pre_activation=True),
    dict(act=na.EP_SIGMOID, add_to=True), dict(add_to=True), dict(),
]


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("M,K,N", [(1, 4096, 1024), (2, 1000, 77), (64, 512, 256)])
@pytest.mark.parametrize("kw", PASS_VARIANTS)
def test_q4_1_linear_bias_epilogue_residual(f16, M, K, N, kw):
    """Linear over q4_1 with a bias, an activation and the residual in both
    orders (an identity epilogue folds it pre-activation, as nnops does)."""
    announce(f"q4_1 linear pass {M}x{K}x{N} f16={f16} {kw}")
    dt = np.float16 if f16 else np.float32
    x = dg.normal(M + 3 * K, (M, K)).astype(dt)
    blk = dg.q4_1_blocks(N + 5, N, K)
    bias = dg.normal(N + 6, (N,)).astype(dt)
    old = dg.normal(N + 7, (M, N)).astype(dt) if kw.get("add_to") else None
    got = run_linear(x, blk, N, gated=False, bias=bias, old=old, **kw)
    act = {None: oracle.ACT_NONE, na.EP_GELU: oracle.ACT_GELU, na.EP_SILU: oracle.ACT_SILU,
           na.EP_RELU: oracle.ACT_RELU, na.EP_SIGMOID: oracle.ACT_SIGMOID}[kw.get("act")]
    active = act != oracle.ACT_NONE or "min_clip" in kw
    pre = kw.get("add_to", False) and (kw.get("residual_pre_activation", False) or not active)
    want = oracle.q4_1_linear(x, blk, N, w_round_f16=q41_f16_weights(M, K, f16), out_f16=f16, bias=bias, out=old,
                              act=act,
                              min_clip=kw.get("min_clip", -math.inf), max_clip=kw.get("max_clip", math.inf),
                              add_to=kw.get("add_to", False), residual_pre=pre).astype(np.float32)
    err = norm_err(got, want)
    assert err <= TOL, err


@pytest.mark.parametrize("M", [1, 40])
def test_q4_1_matmul_bias_gelu_blocks_along_n(M):
    """MatMul over a [K, N] q4_1 weight (blocks along N) with a bias and GELU."""
    import torch
    announce(f"q4_1 matmul kn bias gelu M={M}")
    K, N = 1024, 640
    x = dg.normal(900 + M, (M, K)).astype(np.float32)
    blk = dg.q4_1_blocks(901, K, N)
    bias = dg.normal(902, (N,)).astype(np.float32)
    y = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    op = na.MatMul(transpose_b=False, act=na.EP_GELU)
    ins = [na.tensor(dev(x)), na.tensor(dev(blk), dtype=na.DT_Q4_1, shape=[K, N]), na.tensor(dev(bias))]
    assert op.compute([na.tensor(y)], ins) == na.OK
    torch.cuda.synchronize()
    acc = oracle.gemm_q4_1(x, blk, N, trans_b=False)
    want = oracle.fp_out_pass(acc, N, bias=bias, act=oracle.ACT_GELU)
    assert norm_err(host(y), want) <= TOL


MM_VARIANTS = [
    dict(alpha=0.5, beta=0.75, bias=True),
    dict(alpha=1.0, beta=1.0),
    dict(alpha=2.0, beta=-0.5, act=na.EP_RELU),
    dict(alpha=1.5, beta=3.0, bias=True, act=na.EP_SILU),
    dict(alpha=0.25, beta=0.0, residual_pre=True, bias=True),
]
MM_ACT = {None: oracle.ACT_NONE, na.EP_RELU: oracle.ACT_RELU, na.EP_SILU: oracle.ACT_SILU}


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("M,trans_b", [(1, True), (2, False), (40, True), (300, False)])
@pytest.mark.parametrize("kw", MM_VARIANTS)
def test_q4_1_matmul_alpha_beta(f16, M, trans_b, kw):
    """MatMul's fp epilogue over a q4_1 weight: C = act(alpha P + T(beta C_old
    + bias)) (nnops' order, pinned in tests/test_oracle.py), on the GEMV
    and GEMM routes of both layouts."""
    import torch
    announce(f"q4_1 matmul alpha/beta M={M} trans_b={trans_b} f16={f16} {kw}")
    dt = np.float16 if f16 else np.float32
    K, N = 512, 256
    x = dg.normal(950 + M, (M, K)).astype(dt)
    blk = dg.q4_1_blocks(951, N, K) if trans_b else dg.q4_1_blocks(952, K, N)
    bias = dg.normal(953, (N,)).astype(dt) if kw.get("bias") else None
    old = dg.normal(954, (M, N)).astype(dt)
    y = dev(old)
    op = na.MatMul(transpose_b=trans_b, act=kw.get("act"), alpha=kw["alpha"], beta=kw["beta"],
                   residual_pre_activation=kw.get("residual_pre", False))
    ins = [na.tensor(dev(x)), na.tensor(dev(blk), dtype=na.DT_Q4_1, shape=[N, K] if trans_b else [K, N])]
    if bias is not None:
        ins.append(na.tensor(dev(bias)))
    assert op.compute([na.tensor(y)], ins) == na.OK
    torch.cuda.synchronize()
    acc = oracle.gemm_q4_1(x, blk, N, trans_b=trans_b, w_round_f16=q41_f16_weights(M, K, f16, trans_b, N))
    want = oracle.fp_out_pass(acc, N, out=old, out_f16=f16, bias=bias, act=MM_ACT[kw.get("act")],
                              matmul_order=True, alpha=kw["alpha"], beta=kw["beta"],
                              residual_pre=kw.get("residual_pre", False)).astype(np.float32)
    assert norm_err(host(y).astype(np.float32), want) <= TOL


def test_gated_validation():
    """nnops' gated-form rules (src/ops/linear.cpp:63-107), over a q4_1 weight."""
    import torch
    announce("gated validation")
    M, K, N2 = 2, 64, 64
    x = dev(dg.normal(1, (M, K)).astype(np.float16))
    blk = dev(dg.q4_1_blocks(2, N2, K))
    y = torch.zeros((M, N2 // 2), dtype=torch.float16, device="cuda")
    w = na.tensor(blk, dtype=na.DT_Q4_1, shape=[N2, K])
    ok = na.Linear(gated=True)
    assert ok.validate([na.tensor(x), w], [na.tensor(y)]) == na.OK
    assert na.Linear(gated=True, add_to=True, residual_pre_activation=True).validate(
        [na.tensor(x), w], [na.tensor(y)]) == na.UNSUPPORTED
    assert na.Linear(gated=True, gate_activation=na.EP_LEAKY_RELU).validate(
        [na.tensor(x), w], [na.tensor(y)]) == na.UNSUPPORTED
    y_bad = torch.zeros((M, N2), dtype=torch.float16, device="cuda")
    assert ok.validate([na.tensor(x), w], [na.tensor(y_bad)]) == na.INVALID_ARGUMENT
    w_odd = na.tensor(dev(dg.q4_1_blocks(3, 63, K)), dtype=na.DT_Q4_1, shape=[63, K])
    assert ok.validate([na.tensor(x), w_odd], [na.tensor(y)]) == na.INVALID_ARGUMENT
    s8w = na.tensor(dev(dg.ints(4, (N2, K), -127, 127)))
    assert ok.validate([na.tensor(dev(dg.ints(5, (M, K), -127, 127))), s8w], [na.tensor(y)]) == na.UNSUPPORTED
