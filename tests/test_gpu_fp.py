"""Dense fp MatMul / Linear (f32 x f32, f16 x f16) on the GPU, through the C
ABI (nnops_hip_gemm_fp) and the operator facade, against the oracle: the
float64 sum of the operands' exact products (tests/test_oracle.py pins it to
nnops' own CPU MatMul and Linear), then the fp output pass.

Bars, as the normalized error max|g - w| / max(|w|, rms(w)):
  f32 destination: 2e-5 (f32 accumulation over K <= 4096);
  f16 destination: 2e-3 (one f16 rounding of the output is 2^-11 of it; the
  f32 accumulation before it adds nothing visible)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import datagen as dg
import nnops_amd as na
from gpu_util import dev, host, announce, norm_err

pytestmark = pytest.mark.gpu

TOL = {False: 2e-5, True: 2e-3}

CASES = [
    # GEMV (M <= 16, passes of 4 rows), ragged K / N, unaligned K
    (1, 4096, 1024), (2, 1000, 77), (4, 96, 40), (5, 512, 300), (16, 4096, 256), (3, 37, 19),
    # tile kernel (f32; f16 shapes the ring cannot take) and the f16 ring (split and unsplit)
    (17, 256, 130), (64, 512, 256), (130, 1000, 200), (300, 1024, 520), (512, 4096, 1024), (256, 2048, 4096), (4096, 256, 4096),
]


def run_fp(a, b, trans_b, out_f16, alpha=1.0):
    import torch
    M = a.shape[0]
    n = b.shape[0] if trans_b else b.shape[1]
    c = torch.zeros((M, n), dtype=torch.float16 if out_f16 else torch.float32, device="cuda")
    na.gemm_fp(dev(a), dev(b), c, trans_b=trans_b, alpha=alpha)
    torch.cuda.synchronize()
    return host(c).astype(np.float32)


@pytest.mark.parametrize("M,K,N", CASES)
@pytest.mark.parametrize("trans_b", [True, False])
@pytest.mark.parametrize("f16", [False, True])
def test_gemm_fp(M, K, N, trans_b, f16):
    announce(f"gemm_fp {M}x{K}x{N} trans_b={trans_b} f16={f16}")
    dt = np.float16 if f16 else np.float32
    seed = 7 * M + K + 3 * N + int(trans_b)
    a = dg.normal(seed, (M, K)).astype(dt)
    b = dg.normal(seed + 1, (N, K) if trans_b else (K, N)).astype(dt)
    got = run_fp(a, b, trans_b, f16)
    want = oracle.gemm_fp(a, b, trans_b=trans_b)
    if f16:
        want = want.astype(np.float16).astype(np.float32)
    assert norm_err(got, want) <= TOL[f16]


@pytest.mark.parametrize("M", [1, 300])
def test_gemm_fp_alpha_and_f32_out_from_f16(M):
    """alpha scales the finished sum; f16 operands may write an f32 C."""
    announce(f"gemm_fp alpha M={M}")
    K, N = 512, 256
    a = dg.normal(70 + M, (M, K)).astype(np.float16)
    b = dg.normal(71, (N, K)).astype(np.float16)
    got = run_fp(a, b, True, False, alpha=0.375)
    want = 0.375 * oracle.gemm_fp(a, b, trans_b=True)
    assert norm_err(got, want) <= TOL[False]


def test_gemm_fp_pitched_and_repeat():
    """Pitched A / C rows (the pitch is honoured, padding untouched), two
    calls in a row on the same workspace."""
    import torch
    announce("gemm_fp pitched")
    M, K, N = 320, 1024, 512
    a_full = dg.normal(80, (M, K + 8)).astype(np.float16)
    b = dg.normal(81, (N, K)).astype(np.float16)
    at = dev(a_full)[:, :K]
    c_full = torch.full((M, N + 16), 7.0, dtype=torch.float32, device="cuda")
    c = c_full[:, :N]
    for _ in range(2):
        na.gemm_fp(at, dev(b), c, trans_b=True)
    torch.cuda.synchronize()
    want = oracle.gemm_fp(a_full[:, :K], b, trans_b=True)
    out = host(c_full)
    assert norm_err(out[:, :N], want) <= TOL[False]
    assert np.all(out[:, N:] == 7.0)


MM_KW = [
    dict(),
    dict(bias=True, act=na.EP_RELU),
    dict(alpha=0.5, beta=0.75, bias=True),
    dict(alpha=2.0, beta=1.0, act=na.EP_GELU),
]
MM_ACT = {None: oracle.ACT_NONE, na.EP_RELU: oracle.ACT_RELU, na.EP_GELU: oracle.ACT_GELU}


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("M,trans_b", [(2, False), (3, True), (200, True), (200, False)])
@pytest.mark.parametrize("kw", MM_KW)
def test_matmul_dense(f16, M, trans_b, kw):
    """MatMul over dense operands: the output follows A, the epilogue is
    MatMul's (alpha, bias, beta, activation)."""
    import torch
    announce(f"matmul dense M={M} trans_b={trans_b} f16={f16} {kw}")
    dt = np.float16 if f16 else np.float32
    K, N = 384, 136
    a = dg.normal(90 + M, (M, K)).astype(dt)
    b = dg.normal(91, (N, K) if trans_b else (K, N)).astype(dt)
    bias = dg.normal(92, (N,)).astype(dt) if kw.get("bias") else None
    old = dg.normal(93, (M, N)).astype(dt)
    y = dev(old)
    op = na.MatMul(transpose_b=trans_b, act=kw.get("act"), alpha=kw.get("alpha", 1.0), beta=kw.get("beta", 0.0))
    ins = [na.tensor(dev(a)), na.tensor(dev(b))]
    if bias is not None:
        ins.append(na.tensor(dev(bias)))
    shape, odt = op.output_desc(ins)
    assert shape == [M, N] and odt == (na.DT_F16 if f16 else na.DT_F32)
    assert op.compute([na.tensor(y)], ins) == na.OK
    torch.cuda.synchronize()
    acc = oracle.gemm_fp(a, b, trans_b=trans_b)
    want = oracle.fp_out_pass(acc, N, out=old, out_f16=f16, bias=bias, act=MM_ACT[kw.get("act")],
                              matmul_order=True, alpha=kw.get("alpha", 1.0), beta=kw.get("beta", 0.0))
    assert norm_err(host(y).astype(np.float32), want.astype(np.float32)) <= TOL[f16]


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("M", [1, 4, 96])
@pytest.mark.parametrize("gate", [na.EP_SILU, na.EP_GELU])
def test_linear_gated_dense(f16, M, gate):
    """Linear's gated form over a dense weight of X's type (nnops' own gated
    route, src/ops/linear.cpp:92): W [2N, K], bias [2N] -> [M, N]."""
    import torch
    announce(f"linear gated dense M={M} f16={f16} gate={gate}")
    dt = np.float16 if f16 else np.float32
    K, N = 512, 200
    x = dg.normal(100 + M, (M, K)).astype(dt)
    w = (0.05 * dg.normal(101, (2 * N, K))).astype(dt)
    bias = (0.1 * dg.normal(102, (2 * N,))).astype(dt)
    y = torch.zeros((M, N), dtype=torch.float16 if f16 else torch.float32, device="cuda")
    op = na.Linear(gated=True, gate_activation=gate, gate_limit=7.0)
    ins = [na.tensor(dev(x)), na.tensor(dev(w)), na.tensor(dev(bias))]
    outs = [na.tensor(y)]
    assert op.output_desc(ins)[0] == [M, N]
    assert op.validate(ins, outs) == na.OK
    assert op.compute(outs, ins) == na.OK
    torch.cuda.synchronize()
    g = {na.EP_SILU: oracle.ACT_SILU, na.EP_GELU: oracle.ACT_GELU}[gate]
    want = oracle.fp_linear(x, w, gated=True, gate_act=g, gate_limit=7.0, bias=bias, out_f16=f16)
    assert norm_err(host(y).astype(np.float32), want.astype(np.float32)) <= (4e-3 if f16 else TOL[False])


@pytest.mark.parametrize("f16", [False, True])
def test_linear_dense_bias_residual(f16):
    """Linear over a dense weight with bias, Relu and an add_to residual."""
    import torch
    announce(f"linear dense residual f16={f16}")
    dt = np.float16 if f16 else np.float32
    M, K, N = 40, 256, 96
    x = dg.normal(110, (M, K)).astype(dt)
    w = dg.normal(111, (N, K)).astype(dt)
    bias = dg.normal(112, (N,)).astype(dt)
    old = dg.normal(113, (M, N)).astype(dt)
    y = dev(old)
    op = na.Linear(act=na.EP_RELU, add_to=True)
    assert op.compute([na.tensor(y)], [na.tensor(dev(x)), na.tensor(dev(w)), na.tensor(dev(bias))]) == na.OK
    torch.cuda.synchronize()
    want = oracle.fp_linear(x, w, out_f16=f16, bias=bias, out=old, act=oracle.ACT_RELU, add_to=True)
    assert norm_err(host(y).astype(np.float32), want.astype(np.float32)) <= TOL[f16]


def test_dense_validation():
    """Mixed fp pairs are not a route; the output must follow A."""
    import torch
    announce("dense validation")
    a = dev(dg.normal(1, (4, 64)).astype(np.float16))
    b32 = dev(dg.normal(2, (64, 32)).astype(np.float32))
    b16 = dev(dg.normal(2, (64, 32)).astype(np.float16))
    op = na.MatMul()
    y32 = torch.zeros((4, 32), dtype=torch.float32, device="cuda")
    assert op.compute([na.tensor(y32)], [na.tensor(a), na.tensor(b32)]) == na.UNSUPPORTED
    assert op.compute([na.tensor(y32)], [na.tensor(a), na.tensor(b16)]) == na.INVALID_ARGUMENT


@pytest.mark.parametrize("f16", [False, True])
def test_matmul_dense_batched_broadcast(f16):
    """Batched dense operands with broadcast on leading axes (nnops' batch
    walk): A [2, 1, 70, K] x B [3, K, N] -> [2, 3, 70, N]."""
    import torch
    announce(f"matmul dense broadcast f16={f16}")
    dt = np.float16 if f16 else np.float32
    K, N = 256, 72
    a = dg.normal(120, (2, 1, 70, K)).astype(dt)
    b = dg.normal(121, (3, K, N)).astype(dt)
    out_shape = (2, 3, 70, N)
    c = torch.zeros(out_shape, dtype=torch.float16 if f16 else torch.float32, device="cuda")
    op = na.MatMul()
    ins = [na.tensor(dev(a)), na.tensor(dev(b))]
    shape, _ = op.output_desc(ins)
    assert tuple(shape) == out_shape
    assert op.compute([na.tensor(c)], ins) == na.OK
    torch.cuda.synchronize()
    got = host(c).astype(np.float32)
    for i in range(2):
        for j in range(3):
            want = oracle.gemm_fp(a[i, 0], b[j], trans_b=False)
            if f16:
                want = want.astype(np.float16).astype(np.float32)
            assert norm_err(got[i, j], want) <= TOL[f16]


def test_linear_dense_rank3_input():
    """Linear flattens X's leading dims: X [2, 5, K] x W [N, K] -> [2, 5, N]."""
    import torch
    announce("linear dense rank3")
    K, N = 512, 48
    x = dg.normal(130, (2, 5, K)).astype(np.float16)
    w = dg.normal(131, (N, K)).astype(np.float16)
    y = torch.zeros((2, 5, N), dtype=torch.float16, device="cuda")
    op = na.Linear()
    ins = [na.tensor(dev(x)), na.tensor(dev(w))]
    assert op.output_desc(ins)[0] == [2, 5, N]
    assert op.compute([na.tensor(y)], ins) == na.OK
    torch.cuda.synchronize()
    want = oracle.gemm_fp(x.reshape(10, K), w, trans_b=True).astype(np.float16).astype(np.float32)
    assert norm_err(host(y).astype(np.float32).reshape(10, N), want) <= TOL[True]
