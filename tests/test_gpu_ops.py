"""MatMul / Linear through the operator C facade on the GPU: the C++ front end's
routing of QuantParams (host tables staged into the workspace, device tables
read in place), the epilogue's Requantize table, batch broadcast, Linear's
leading-dim flattening, s8 add_to, and the workspace contract."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import datagen as dg
import nnops_amd as na
from gpu_util import dev, host, announce, pitched

pytestmark = pytest.mark.gpu


def test_matmul_s8_host_and_device_tables():
    import torch
    announce("matmul host/device tables")
    M, K, N = 37, 300, 90
    a = dg.act_s8(1, (M, K))
    b = dg.ints(2, (K, N), -127, 127)
    sb = dg.uniform(3, (N,), 0.001, 0.01)
    zb = dg.ints(4, (N,), -2, 2, np.int32)
    bias = dg.ints(5, (N,), -3000, 3000, np.int32)
    want = oracle.gemm_i8(a, b, bias=bias, out_kind=oracle.OUT_S8, s_a=0.02, s_b=sb, zp_b=zb,
                          s_out=0.2, zp_out=-3, act=oracle.ACT_RELU)
    for device_tables in (False, True):
        da, db, dbias = dev(a), dev(b), dev(bias)
        c = torch.zeros((M, N), dtype=torch.int8, device="cuda")
        op = na.MatMul(output_dtype=na.DT_S8, act=na.EP_RELU)
        sbt = dev(sb) if device_tables else sb
        zbt = dev(zb) if device_tables else zb
        ins = [na.tensor(da, scale=0.02), na.tensor(db, scale_data=sbt, zero_point_data=zbt, granularity=2),
               na.tensor(dbias)]
        outs = [na.tensor(c, scale=0.2, zero_point=-3)]
        assert op.validate(ins, outs) == na.OK
        assert op.compute(outs, ins) == na.OK
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(c), want)


def test_matmul_requant_table_and_batch_broadcast():
    import torch
    announce("matmul batch + requant table")
    Bt, M, K, N = 3, 20, 128, 48
    a = dg.ints(11, (Bt, M, K), -127, 127)
    b = dg.ints(12, (K, N), -127, 127)  # broadcast over the batch
    so = dg.uniform(13, (M,), 50.0, 200.0)
    c = torch.zeros((Bt, M, N), dtype=torch.int8, device="cuda")
    op = na.MatMul(output_dtype=na.DT_S8, quant=na.EQ_REQUANTIZE, quant_scales=so, quant_param_count=M)
    ins = [na.tensor(dev(a)), na.tensor(dev(b))]
    outs = [na.tensor(c)]
    shape, dt = op.output_desc(ins)
    assert shape == [Bt, M, N] and dt == na.DT_S8
    assert op.compute(outs, ins) == na.OK
    torch.cuda.synchronize()
    got = host(c)
    for i in range(Bt):
        want = oracle.gemm_i8(a[i], b, out_kind=oracle.OUT_S8, s_out_rows=so)
        np.testing.assert_array_equal(got[i], want)


def test_linear_rank3_s32_and_missing_workspace():
    import torch
    announce("linear rank3")
    X = dg.ints(21, (2, 9, 64), -127, 127)
    W = dg.ints(22, (40, 64), -127, 127)
    y = torch.zeros((2, 9, 40), dtype=torch.int32, device="cuda")
    op = na.Linear(output_dtype=na.DT_S32)
    ins = [na.tensor(dev(X)), na.tensor(dev(W))]
    outs = [na.tensor(y)]
    assert op.compute(outs, ins) == na.OK
    torch.cuda.synchronize()
    want = oracle.gemm_i8(X.reshape(18, 64), W, trans_b=True).reshape(2, 9, 40)
    np.testing.assert_array_equal(host(y), want)
    # a [K,N] MatMul needs workspace: a null workspace is not_initialized, nothing written
    y2 = torch.full((9, 40), 77, dtype=torch.int32, device="cuda")
    op2 = na.MatMul(output_dtype=na.DT_S32)
    Wt = np.ascontiguousarray(W.T)
    assert op2.compute([na.tensor(y2)], [na.tensor(dev(X[0])), na.tensor(dev(Wt))], workspace=0) \
        == na.NOT_INITIALIZED
    torch.cuda.synchronize()
    assert (host(y2) == 77).all()


def test_linear_s8_add_to_gelu_config5_shape_small():
    """Config 5's route at a reduced M (full shape runs in the bench): Linear
    over a [K,N]-stored weight is expressed as MatMul(transpose_b=False) with
    the float epilogue; here Linear's own [N,K] form is used."""
    import torch
    announce("linear add_to gelu")
    M, K, N = 33, 1440, 256
    x = dg.act_s8(31, (M, K))
    w = dg.ints(32, (N, K), -127, 127)
    sb = dg.uniform(33, (N,), 0.001, 0.01)
    bias = dg.ints(34, (N,), -5000, 5000, np.int32)
    c0 = dg.ints(35, (M, N), -128, 127)
    xt = pitched(x, K + 64)
    yt = pitched(c0, N + 64)
    op = na.Linear(output_dtype=na.DT_S8, act=na.EP_GELU, add_to=True)
    ins = [na.tensor(xt, scale=0.02), na.tensor(dev(w), scale_data=sb, granularity=2), na.tensor(dev(bias))]
    outs = [na.tensor(yt, scale=2.0, zero_point=1)]
    assert op.compute(outs, ins) == na.OK
    torch.cuda.synchronize()
    want = oracle.gemm_i8(x, w, trans_b=True, bias=bias, out_kind=oracle.OUT_S8, s_a=0.02, s_b=sb,
                          s_out=2.0, zp_out=1, float_ep=True, act=oracle.ACT_GELU, add_to=True,
                          c=c0.copy())
    np.testing.assert_array_equal(host(yt), want)


def test_linear_q4_1_f16():
    import torch
    announce("linear q4_1")
    M, K, N = 1, 4096, 512
    x = dg.normal(41, (M, K)).astype(np.float16)
    blk = dg.q4_1_blocks(42, N, K)
    y = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    op = na.Linear()
    ins = [na.tensor(dev(x)), na.tensor(dev(blk), dtype=na.DT_Q4_1, shape=[N, K])]
    shape, dt = op.output_desc(ins)
    assert shape == [M, N] and dt == na.DT_F16
    assert op.compute([na.tensor(y)], ins) == na.OK
    torch.cuda.synchronize()
    want = oracle.gemm_q4_1(x, blk, N, trans_b=True)
    from gpu_util import norm_err
    assert norm_err(host(y), want) <= 2e-3


def test_linear_from_gguf_q4_1_and_i8(tmp_path):
    """A GGUF file's Q4_1 and I8 tensors, read through the memory map and
    uploaded, drive Linear directly (the [N][K/32] block rows are the Linear
    weight form)."""
    import torch
    from nnops_amd import gguf
    announce("linear from gguf")
    M, K, N = 3, 1024, 200
    blk = dg.q4_1_blocks(121, N, K)
    w8 = dg.ints(122, (N, K), -127, 127)
    p = str(tmp_path / "m.gguf")
    gguf.write_gguf(p, {"q": (gguf.GGML_Q4_1, (K, N), blk.tobytes()), "i": (gguf.GGML_I8, (K, N), w8.tobytes())})
    g = gguf.open_gguf(p)
    wq, dtq, (n, k) = gguf.load_weight(g, "q")
    wi, dti, _ = gguf.load_weight(g, "i")
    g.close()
    assert (n, k) == (N, K) and dtq == na.DT_Q4_1 and dti == na.DT_S8
    x = dg.normal(123, (M, K)).astype(np.float16)
    y = torch.zeros((M, N), dtype=torch.float16, device="cuda")
    assert na.Linear().compute([na.tensor(y)], [na.tensor(dev(x)), na.tensor(wq, dtype=dtq, shape=[N, K])]) == na.OK
    xs = dg.act_s8(124, (M, K))
    yi = torch.zeros((M, N), dtype=torch.int32, device="cuda")
    assert na.Linear(output_dtype=na.DT_S32).compute([na.tensor(yi)], [na.tensor(dev(xs)), na.tensor(wi)]) == na.OK
    torch.cuda.synchronize()
    want = oracle.gemm_q4_1(x, blk, N, trans_b=True, w_round_f16=True, c_f16=True).astype(np.float32)
    from gpu_util import norm_err
    assert norm_err(host(y).astype(np.float32), want) <= 2e-3
    np.testing.assert_array_equal(host(yi), oracle.gemm_i8(xs, w8, trans_b=True))


def test_matmul_rank6_broadcast():
    """Rank-6 operands with broadcast on several leading axes (nnops' batch
    walk, matmul_internal.h:90-151; its CUDA ceiling is rank 6)."""
    import torch
    announce("matmul rank6")
    a_shape = (2, 1, 3, 1, 5, 64)
    b_shape = (1, 2, 1, 2, 64, 24)
    a = dg.ints(131, a_shape, -127, 127)
    b = dg.ints(132, b_shape, -127, 127)
    out_shape = (2, 2, 3, 2, 5, 24)
    c = torch.zeros(out_shape, dtype=torch.int32, device="cuda")
    op = na.MatMul()
    ins = [na.tensor(dev(a)), na.tensor(dev(b))]
    shape, dt = op.output_desc(ins)
    assert tuple(shape) == out_shape
    assert op.compute([na.tensor(c)], ins) == na.OK
    torch.cuda.synchronize()
    got = host(c)
    for idx in np.ndindex(*out_shape[:-2]):
        ia = tuple(i if d > 1 else 0 for i, d in zip(idx, a_shape[:-2]))
        ib = tuple(i if d > 1 else 0 for i, d in zip(idx, b_shape[:-2]))
        np.testing.assert_array_equal(got[idx], oracle.gemm_i8(np.ascontiguousarray(a[ia]),
                                                               np.ascontiguousarray(b[ib])))


def test_linear_rank1_input_f32_out():
    """A rank-1 X is one row over the same buffers (nnops' linear.cpp:234-246)."""
    import torch
    announce("linear rank1")
    K, N = 640, 96
    x = dg.act_s8(141, (K,))
    w = dg.ints(142, (N, K), -127, 127)
    bias = dg.normal(143, (N,)).astype(np.float32)
    y = torch.zeros((N,), dtype=torch.float32, device="cuda")
    op = na.Linear(output_dtype=na.DT_F32, act=na.EP_RELU)
    ins = [na.tensor(dev(x), scale=0.03), na.tensor(dev(w), scale=0.002), na.tensor(dev(bias))]
    shape, dt = op.output_desc(ins)
    assert shape == [N] and dt == na.DT_F32
    assert op.compute([na.tensor(y)], ins) == na.OK
    torch.cuda.synchronize()
    want = oracle.gemm_i8(x.reshape(1, K), w, trans_b=True, out_kind=oracle.OUT_F32, bias=bias, s_a=0.03, s_b=0.002,
                          act=oracle.ACT_RELU).reshape(N)
    np.testing.assert_array_equal(host(y).view(np.uint32), want.view(np.uint32))
