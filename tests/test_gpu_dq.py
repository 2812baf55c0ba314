"""Dequantizing destinations, the fp-activation int8 MatMul, and
QuantizeLinear / DequantizeLinear on the GPU, against the CPU oracle (itself
pinned bit for bit to the compiled reference's matmul_dq_ref and to the known
answers of the reference's quant_linear tests).

Bars:
  - integer arithmetic, the dequantize multiply, bias, residual, clip and the
    piecewise-linear activations (none, relu, relu6, leaky relu, hardswish):
    bit-exact in f32 and f16;
  - activations through exp / tanh (gelu, sigmoid, tanh, silu, elu): the device
    library's expf / tanhf against glibc's, within 8 f32 ulps of the oracle
    (f32 out) or 1 f16 ulp (f16 out), the double rounding to f16 allowing a
    one-ulp flip, plus 2^-22 absolute for GELU's cancellation near zero;
  - QuantizeLinear / DequantizeLinear: bit-exact."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import datagen as dg
import nnops_amd as na
from gpu_util import dev, host, announce, pitched

pytestmark = pytest.mark.gpu

EXACT_ACTS = (na.ACT_NONE, na.ACT_RELU, na.ACT_RELU6, na.ACT_LEAKY_RELU, na.ACT_HARDSWISH)
TRANSC_ACTS = (na.ACT_GELU, na.ACT_SIGMOID, na.ACT_TANH, na.ACT_SILU, na.ACT_ELU)


def check(got, want, act):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.dtype == want.dtype and got.shape == want.shape
    if act in EXACT_ACTS:
        ui = np.uint16 if got.dtype == np.float16 else np.uint32
        bad = got.view(ui) != want.view(ui)
        assert not bad.any(), (np.argwhere(bad)[:5], got[bad][:5], want[bad][:5])
        return
    # 2^-22 absolute covers the cancellation in GELU's 1 + tanh(u) near -1,
    # where one ulp of tanh is large against the result
    if got.dtype == np.float16:
        tol = np.spacing(np.abs(want)).astype(np.float64) + 2.0 ** -22
    else:
        tol = 8 * np.spacing(np.abs(want)).astype(np.float64) + 2.0 ** -22
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert (err <= tol).all(), float((err / np.maximum(tol, 1e-45)).max())


def run_dq(a, b, *, trans_b, out16, bias=None, s_a=0.02, zp_a=0, s_b=0.01, zp_b=0, act=na.ACT_NONE,
           alpha=0.1, beta=1.0, lo=-np.inf, hi=np.inf, add_to=False, residual_pre=False, c0=None,
           ldc=None):
    import torch
    M = a.shape[0]
    N = b.shape[0] if trans_b else b.shape[1]
    odt = np.float16 if out16 else np.float32
    if c0 is None:
        c0 = np.zeros((M, N), odt)
    dc = pitched(c0, ldc) if ldc else dev(c0)

    def sd(x):
        return dev(x) if isinstance(x, np.ndarray) else x
    na.gemm_i8(dev(a), dev(b), dc, trans_b=trans_b, out_kind=na.OUT_F16 if out16 else na.OUT_F32,
               bias_fp=None if bias is None else dev(bias), s_a=sd(s_a), zp_a=sd(zp_a), s_b=sd(s_b),
               zp_b=sd(zp_b), act=act, act_alpha=alpha, act_beta=beta, min_clip=lo, max_clip=hi,
               add_to=add_to, residual_pre=residual_pre)
    torch.cuda.synchronize()
    got = host(dc)
    want = oracle.gemm_i8(a, b, trans_b=trans_b, out_kind=oracle.OUT_F16 if out16 else oracle.OUT_F32,
                          bias=bias, s_a=s_a, zp_a=zp_a, s_b=s_b, zp_b=zp_b, act=act, act_alpha=alpha,
                          act_beta=beta, min_clip=lo, max_clip=hi, add_to=add_to,
                          residual_pre=residual_pre, c=c0.copy())
    return got, want


# every dispatch route of the int8 GEMM: [K,N] column GEMV (M <= 2), row GEMV
# (M <= 4), small-M MFMA GEMV (M <= 16), ring GEMM (with K splits and the
# reduce / output pass), the general MFMA GEMM
SHAPES = [(1, 512, 96), (2, 4096, 1008), (3, 100, 37), (12, 1024, 2048), (16, 512, 130),
          (100, 1000, 333), (300, 512, 257), (333, 2048, 512), (1024, 512, 4096)]


@pytest.mark.parametrize("M,K,N", SHAPES)
@pytest.mark.parametrize("trans_b", [True, False])
@pytest.mark.parametrize("out16", [False, True])
def test_dq_routes_bias_per_channel(M, K, N, trans_b, out16):
    announce(f"dq {M}x{K}x{N} tb={trans_b} f16={out16}")
    seed = M + 7 * K + 13 * N + 2 * trans_b + out16
    a = dg.act_s8(seed, (M, K))
    b = dg.ints(seed + 1, (N, K) if trans_b else (K, N), -127, 127)
    sa = dg.uniform(seed + 2, (M,), 0.01, 0.03)
    zpa = dg.ints(seed + 3, (M,), -4, 4, np.int32)
    sb = dg.uniform(seed + 4, (N,), 0.001, 0.01)
    zpb = dg.ints(seed + 5, (N,), -2, 2, np.int32)
    bias = dg.normal(seed + 6, (N,)).astype(np.float16 if out16 else np.float32)
    got, want = run_dq(a, b, trans_b=trans_b, out16=out16, bias=bias, s_a=sa, zp_a=zpa, s_b=sb, zp_b=zpb)
    check(got, want, na.ACT_NONE)


@pytest.mark.parametrize("act", EXACT_ACTS + TRANSC_ACTS)
@pytest.mark.parametrize("M,K,N", [(2, 1024, 300), (64, 256, 200), (520, 1024, 512)])
@pytest.mark.parametrize("out16", [False, True])
def test_dq_activations_and_clip(act, M, K, N, out16):
    announce(f"dq act={act} {M}x{K}x{N} f16={out16}")
    seed = 100 * act + M + N + out16
    a = dg.act_s8(seed, (M, K))
    b = dg.ints(seed + 1, (N, K), -127, 127)
    bias = dg.normal(seed + 2, (N,)).astype(np.float16 if out16 else np.float32)
    got, want = run_dq(a, b, trans_b=True, out16=out16, bias=bias, s_a=0.02, s_b=0.002, act=act,
                       alpha=0.07, beta=0.8, lo=-3.0, hi=4.5)
    check(got, want, act)


@pytest.mark.parametrize("residual_pre", [True, False])
@pytest.mark.parametrize("out16", [False, True])
@pytest.mark.parametrize("M,K,N", [(1, 512, 200), (40, 640, 96), (700, 512, 640)])
def test_dq_residual_pre_and_post(residual_pre, out16, M, K, N):
    announce(f"dq residual pre={residual_pre} f16={out16} {M}x{K}x{N}")
    seed = 5 * M + N + residual_pre + 2 * out16
    a = dg.act_s8(seed, (M, K))
    b = dg.ints(seed + 1, (N, K), -127, 127)
    c0 = dg.normal(seed + 2, (M, N)).astype(np.float16 if out16 else np.float32)
    got, want = run_dq(a, b, trans_b=True, out16=out16, s_a=0.02, s_b=0.003, act=na.ACT_RELU,
                       add_to=True, residual_pre=residual_pre, c0=c0, ldc=N + 24)
    check(got, want, na.ACT_RELU)


# --- through the operator API ----------------------------------------------------

@pytest.mark.parametrize("out_dt", [na.DT_F32, na.DT_F16])
def test_linear_dq_add_to_post_activation(out_dt):
    """Linear, int8 pair, f32/f16 destination, add_to after a HardSwish
    epilogue (the f16 route rounds the activation to f16 before the add)."""
    import torch
    announce(f"linear dq add_to post dt={out_dt}")
    M, K, N = 45, 768, 160
    f16 = out_dt == na.DT_F16
    npdt = np.float16 if f16 else np.float32
    x = dg.act_s8(41, (M, K))
    w = dg.ints(42, (N, K), -127, 127)
    sb = dg.uniform(43, (N,), 0.001, 0.01)
    bias = dg.normal(44, (N,)).astype(npdt)
    c0 = dg.normal(45, (M, N)).astype(npdt)
    y = dev(c0)
    op = na.Linear(output_dtype=out_dt, act=na.EP_HARDSWISH, act_beta=0.9, add_to=True)
    ins = [na.tensor(dev(x), scale=0.02), na.tensor(dev(w), scale_data=sb, granularity=2),
           na.tensor(dev(bias))]
    assert op.compute([na.tensor(y)], ins) == na.OK
    torch.cuda.synchronize()
    want = oracle.gemm_i8(x, w, trans_b=True, out_kind=oracle.OUT_F16 if f16 else oracle.OUT_F32,
                          bias=bias, s_a=0.02, s_b=sb, act=oracle.ACT_HARDSWISH, act_beta=0.9,
                          add_to=True, residual_pre=False, c=c0.copy())
    check(host(y), want, na.ACT_HARDSWISH)


def test_linear_dq_add_to_identity_folds_pre():
    """An identity epilogue folds the residual into the sum (no f16 rounding of
    the product first), as nnops' Linear does."""
    import torch
    announce("linear dq add_to identity")
    M, K, N = 9, 256, 72
    x = dg.act_s8(51, (M, K))
    w = dg.ints(52, (N, K), -127, 127)
    c0 = dg.normal(53, (M, N)).astype(np.float16)
    y = dev(c0)
    op = na.Linear(output_dtype=na.DT_F16, add_to=True)
    assert op.compute([na.tensor(y)], [na.tensor(dev(x), scale=0.05), na.tensor(dev(w), scale=0.004)]) == na.OK
    torch.cuda.synchronize()
    want = oracle.gemm_i8(x, w, trans_b=True, out_kind=oracle.OUT_F16, s_a=0.05, s_b=0.004,
                          add_to=True, residual_pre=True, c=c0.copy())
    check(host(y), want, na.ACT_NONE)


def fp_a_want(a, b, *, trans_b, s_a, zp_a, s_b, zp_b, bias, act, act_u8, lo=-np.inf, hi=np.inf,
              alpha=0.0, beta=1.0):
    M = a.shape[0]
    sa = np.broadcast_to(np.asarray(s_a, np.float32), (M,))
    za = np.broadcast_to(np.asarray(zp_a), (M,))
    aq = oracle.quantize_linear(a, sa, za, out_dtype=np.uint8 if act_u8 else np.int8, axis=-1)
    out = oracle.OUT_F16 if a.dtype == np.float16 else oracle.OUT_F32
    return oracle.gemm_i8(aq, b, trans_b=trans_b, out_kind=out, s_a=sa, zp_a=za.astype(np.int32),
                          s_b=s_b, zp_b=zp_b, bias=bias, act=act, min_clip=lo, max_clip=hi,
                          act_alpha=alpha, act_beta=beta)


@pytest.mark.parametrize("M,K,N", [(1, 4096, 512), (7, 300, 129), (64, 1024, 256), (512, 2048, 1024)])
@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("per_token", [False, True])
@pytest.mark.parametrize("act_u8", [False, True])
def test_matmul_fp_activation_s8_weight(M, K, N, f16, per_token, act_u8):
    """MatMul: f32/f16 A with offline per-tensor / per-token QuantParams x s8
    B -> A's dtype (quantize A, int8 GEMM, dequantize)."""
    import torch
    announce(f"fp-A matmul {M}x{K}x{N} f16={f16} tok={per_token} u8={act_u8}")
    seed = M + K + N + 2 * f16 + 4 * per_token + 8 * act_u8
    npdt = np.float16 if f16 else np.float32
    a = dg.normal(seed, (M, K), 2.0).astype(npdt)
    b = dg.ints(seed + 1, (K, N), -127, 127)
    if per_token:
        s_a = dg.uniform(seed + 2, (M,), 0.01, 0.03)
        zp_a = dg.ints(seed + 3, (M,), 120, 136, np.int32) if act_u8 else dg.ints(seed + 3, (M,), -5, 5, np.int32)
    else:
        s_a, zp_a = 0.02, (128 if act_u8 else 0)
    sb = dg.uniform(seed + 4, (N,), 0.001, 0.01)
    bias = dg.normal(seed + 5, (N,)).astype(npdt)
    c = torch.zeros((M, N), dtype=torch.float16 if f16 else torch.float32, device="cuda")
    op = na.MatMul(act=na.EP_RELU, act_quant_dtype=na.DT_U8 if act_u8 else na.DT_S8)
    if per_token:
        ta = na.tensor(dev(a), scale_data=s_a, zero_point_data=zp_a, granularity=1)
    else:
        ta = na.tensor(dev(a), scale=s_a, zero_point=zp_a)
    ins = [ta, na.tensor(dev(b), scale_data=sb, granularity=2), na.tensor(dev(bias))]
    shape, dt = op.output_desc(ins)
    assert shape == [M, N] and dt == (na.DT_F16 if f16 else na.DT_F32)
    assert op.compute([na.tensor(c)], ins) == na.OK
    torch.cuda.synchronize()
    want = fp_a_want(a, b, trans_b=False, s_a=s_a, zp_a=zp_a, s_b=sb, zp_b=0, bias=bias,
                     act=oracle.ACT_RELU, act_u8=act_u8)
    check(host(c), want, na.ACT_RELU)


def test_matmul_fp_activation_batched_per_token_global_rows():
    """Batched A [B, M, K] with per-token tables over all B*M rows: each batch
    reads its own rows (nnops indexes per-token arrays by A's global row)."""
    import torch
    announce("fp-A matmul batched per-token")
    Bt, M, K, N = 3, 10, 256, 64
    a = dg.normal(61, (Bt, M, K), 2.0).astype(np.float32)
    b = dg.ints(62, (K, N), -127, 127)
    s_a = dg.uniform(63, (Bt * M,), 0.01, 0.03)
    zp_a = dg.ints(64, (Bt * M,), -5, 5, np.int32)
    c = torch.zeros((Bt, M, N), dtype=torch.float32, device="cuda")
    op = na.MatMul()
    ins = [na.tensor(dev(a), scale_data=s_a, zero_point_data=zp_a, granularity=1),
           na.tensor(dev(b), scale=0.004)]
    assert op.compute([na.tensor(c)], ins) == na.OK
    torch.cuda.synchronize()
    got = host(c)
    for i in range(Bt):
        rows = slice(i * M, (i + 1) * M)
        want = fp_a_want(a[i], b, trans_b=False, s_a=s_a[rows], zp_a=zp_a[rows], s_b=0.004, zp_b=0,
                         bias=None, act=oracle.ACT_NONE, act_u8=False)
        check(got[i], want, na.ACT_NONE)


def test_matmul_fp_activation_rejects():
    import torch
    announce("fp-A matmul rejects")
    a = dev(np.ones((4, 64), np.float32))
    b = dev(np.ones((64, 8), np.int8))
    c = torch.zeros((4, 8), dtype=torch.float32, device="cuda")
    # inactive QuantParams: no defined semantics
    assert na.MatMul().compute([na.tensor(c)], [na.tensor(a), na.tensor(b)]) == na.INVALID_ARGUMENT
    # transpose_a is outside the route
    at = dev(np.ones((64, 4), np.float32))
    assert na.MatMul(transpose_a=True).compute([na.tensor(c)], [na.tensor(at, scale=0.1), na.tensor(b)]) \
        == na.UNSUPPORTED
    # Linear has no fp-activation x s8 route
    w = dev(np.ones((8, 64), np.int8))
    assert na.Linear().compute([na.tensor(c)], [na.tensor(a, scale=0.1), na.tensor(w)]) == na.UNSUPPORTED


# --- QuantizeLinear / DequantizeLinear ---------------------------------------

def qdq_case(shape, n_params, axis, seed, zp_u8):
    scale = dg.uniform(seed, (n_params,), 0.01, 0.2)
    if zp_u8:
        zp = dg.ints(seed + 1, (n_params,), 100, 156, np.uint8)
    else:
        zp = dg.ints(seed + 1, (n_params,), -10, 10, np.int8)
    return scale, zp


QDQ_CASES = [
    # (shape, n_params, axis)
    ((1000,), 1, -1), ((37, 101), 1, -1), ((37, 101), 37, -1), ((5, 6, 33), 30, -1),
    ((64, 4096), 64, -1), ((3, 7, 40), 7, 1), ((16, 24), 16, 0), ((2, 5, 3, 17), 3, 2),
    ((4096, 4096), 4096, -1), ((4096, 4096), 1, -1), ((1,), 1, -1),
]


@pytest.mark.parametrize("shape,n_params,axis", QDQ_CASES)
@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("u8", [False, True])
def test_quantize_dequantize_linear(shape, n_params, axis, f16, u8):
    import torch
    announce(f"qdq {shape} p={n_params} axis={axis} f16={f16} u8={u8}")
    seed = sum(shape) + n_params + 3 * f16 + 5 * u8
    npdt = np.float16 if f16 else np.float32
    x = (dg.normal(seed, shape, 1.0) * 8).astype(npdt)
    if x.size > 8:
        with np.errstate(over="ignore"):   # 1e5 is inf in f16 too
            x.ravel()[:4] = np.array([np.nan, np.inf, -np.inf, 1e5], np.float32).astype(npdt)
    scale, zp = qdq_case(shape, n_params, axis, seed + 10, u8)
    qdt = na.DT_U8 if u8 else na.DT_S8
    q = torch.zeros(shape, dtype=torch.uint8 if u8 else torch.int8, device="cuda")
    op = na.QuantizeLinear(axis=axis, output_dtype=qdt)
    ins = [na.tensor(dev(x)), na.tensor(dev(scale)), na.tensor(dev(zp))]
    oshape, odt = op.output_desc(ins)
    assert oshape == list(shape) and odt == qdt
    assert op.validate(ins, [na.tensor(q)]) == na.OK
    assert op.compute([na.tensor(q)], ins) == na.OK
    y = torch.zeros(shape, dtype=torch.float16 if f16 else torch.float32, device="cuda")
    dop = na.DequantizeLinear(axis=axis, output_dtype=na.DT_F16 if f16 else na.DT_F32)
    assert dop.compute([na.tensor(y)], [na.tensor(q), na.tensor(dev(scale)), na.tensor(dev(zp))]) == na.OK
    torch.cuda.synchronize()
    want_q = oracle.quantize_linear(x, scale, zp.astype(np.int32), out_dtype=np.uint8 if u8 else np.int8,
                                    axis=axis)
    gq = host(q)
    assert np.array_equal(gq, want_q), np.argwhere(gq != want_q)[:5]
    want_y = oracle.dequantize_linear(want_q, scale, zp.astype(np.int32), out_dtype=npdt, axis=axis)
    gy = host(y)
    ui = np.uint16 if f16 else np.uint32
    assert np.array_equal(gy.view(ui), want_y.view(ui)), np.argwhere(gy.view(ui) != want_y.view(ui))[:5]


@pytest.mark.parametrize("cols", [1024, 1000])
def test_dequantize_f16_rounds_twice(cols):
    """y = fma(q, s, -zp * s) is rounded to f32 and then to f16, as the
    reference does: q = -128, s = 0.11721731722354889, zp = 3 gives an f32
    value whose single rounding to f16 lands one ulp away (a fused
    mixed-precision fma would). The rows kernel (1024 | cols) and the
    general one (cols = 1000)."""
    import torch
    announce(f"dequantize f16 double rounding cols={cols}")
    rows = 8
    q = np.full((rows, cols), -128, np.int8)
    q[:, 1::2] = dg.ints(77, (rows, cols // 2), -128, 127, np.int8)
    scale = np.full((rows,), 0.11721731722354889, np.float32)
    zp = np.full((rows,), 3, np.int8)
    y = torch.zeros((rows, cols), dtype=torch.float16, device="cuda")
    dop = na.DequantizeLinear(axis=-1, output_dtype=na.DT_F16)
    assert dop.compute([na.tensor(y)], [na.tensor(dev(q)), na.tensor(dev(scale)), na.tensor(dev(zp))]) == na.OK
    torch.cuda.synchronize()
    want = oracle.dequantize_linear(q, scale, zp.astype(np.int32), out_dtype=np.float16, axis=-1)
    assert want[0, 0].view(np.uint16) == 0xcbae
    np.testing.assert_array_equal(host(y).view(np.uint16), want.view(np.uint16))


def test_quant_linear_rejects():
    import torch
    announce("qdq rejects")
    x = dev(np.ones((4, 8), np.float32))
    s = dev(np.ones(4, np.float32))
    z = dev(np.zeros(4, np.int8))
    q = torch.zeros((4, 8), dtype=torch.int8, device="cuda")
    op = na.QuantizeLinear(axis=-1)
    # wrong zero-point dtype / scale dtype
    assert op.compute([na.tensor(q)], [na.tensor(x), na.tensor(s), na.tensor(dev(np.zeros(4, np.int32)))]) \
        == na.INVALID_ARGUMENT
    assert op.compute([na.tensor(q)], [na.tensor(x), na.tensor(dev(np.ones(4, np.float16))), na.tensor(z)]) \
        == na.INVALID_ARGUMENT
    # per-token scale count must equal the number of rows
    s3 = dev(np.ones(3, np.float32))
    z3 = dev(np.zeros(3, np.int8))
    assert op.compute([na.tensor(q)], [na.tensor(x), na.tensor(s3), na.tensor(z3)]) == na.INVALID_ARGUMENT
    # a pitched (non-compact) view is not a route
    xp = pitched(np.ones((4, 8), np.float32), 16)
    assert op.compute([na.tensor(q)], [na.tensor(xp), na.tensor(s), na.tensor(z)]) == na.UNSUPPORTED
    # an integer dequantize request resolves to f32
    d = na.DequantizeLinear(output_dtype=na.DT_S8)
    _, dt = d.output_desc([na.tensor(q), na.tensor(s), na.tensor(z)])
    assert dt == na.DT_F32


@pytest.mark.parametrize("out16", [False, True])
@pytest.mark.parametrize("act", [na.ACT_NONE, na.ACT_RELU])
@pytest.mark.parametrize("add_to,residual_pre", [(False, False), (True, True), (True, False)])
@pytest.mark.parametrize("M,N", [(1024, 1024), (1000, 1020)])
def test_dq_fused_ring_output_pass(out16, act, add_to, residual_pre, M, N):
    """Shapes whose ring GEMM runs unsplit take the fused dequantizing output
    pass (no partials): per-token s_a, per-channel s_b, bias, clip, Relu,
    pre/post residual, against the oracle bit for bit."""
    announce(f"dq fused ring f16={out16} act={act} add_to={add_to} pre={residual_pre} M={M} N={N}")
    K = 512
    seed = 900 + 2 * out16 + 4 * act + 8 * add_to + 16 * residual_pre
    a = dg.act_s8(seed, (M, K))
    b = dg.ints(seed + 1, (N, K), -127, 127)
    sa = dg.uniform(seed + 2, (M,), 0.01, 0.03)
    sb = dg.uniform(seed + 3, (N,), 0.001, 0.01)
    bias = dg.normal(seed + 4, (N,)).astype(np.float16 if out16 else np.float32)
    c0 = dg.normal(seed + 5, (M, N)).astype(np.float16 if out16 else np.float32)
    got, want = run_dq(a, b, trans_b=True, out16=out16, bias=bias, s_a=sa, s_b=sb, act=act, lo=-2.5, hi=3.0,
                       add_to=add_to, residual_pre=residual_pre, c0=c0)
    check(got, want, act)
