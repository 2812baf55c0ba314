"""The QuantizeLinear / DequantizeLinear oracle pinned against the known answers
of the reference's tests/test_quant_linear.cpp and against float64 arithmetic
that fixes each rounding step independently of the oracle's own formula."""
from __future__ import annotations

import numpy as np
import pytest

import oracle

Q = oracle.quantize_linear
DQ = oracle.dequantize_linear
f32 = np.float32


# --- known answers: tests/test_quant_linear.cpp ------------------------------

def test_quantize_known_per_tensor():  # test_quant_linear.cpp:35-196
    assert Q(np.array([0, 1, 2], f32), 1.0, 0).tolist() == [0, 1, 2]
    assert Q(np.array([0, 2, 4], f32), 2.0, 0).tolist() == [0, 1, 2]
    assert Q(np.array([0, 1, 2], f32), 1.0, 100).tolist() == [100, 101, 102]
    assert Q(np.array([0, 200, -200], f32), 1.0, 0).tolist() == [0, 127, -128]
    assert Q(np.array([-1, 0, 1, 300], f32), 1.0, 0, out_dtype=np.uint8).tolist() == [0, 0, 1, 255]
    assert Q(np.array([0, 1, -1], f32), 1.0, 128, out_dtype=np.uint8).tolist() == [128, 129, 127]


def test_quantize_known_per_channel_ties_to_even():  # :198-226
    x = np.array([[0, 1, 2], [10, 11, 12]], f32)
    got = Q(x, [1, 2, 3], [0, 0, 0], axis=1)
    assert got.ravel().tolist() == [0, 0, 1, 10, 6, 4]


def test_quantize_known_per_token():  # :228-294
    x = np.array([[0, 1, 2], [10, 20, 30]], f32)
    assert Q(x, [1, 10], [0, 0], axis=-1).ravel().tolist() == [0, 1, 2, 1, 2, 3]
    x3 = np.array([0, 1, 2, 4, 10, 20, 30, 40], f32).reshape(2, 2, 2)
    assert Q(x3, [1, 2, 5, 10], [0] * 4, axis=-1).ravel().tolist() == [0, 1, 1, 2, 2, 4, 3, 4]


def test_quantize_known_axis0_weights():  # :296-328
    x = np.array([[0, 1, 2, 3], [10, 20, 30, 40]], f32)
    assert Q(x, [1, 10], [0, 0], axis=0).ravel().tolist() == [0, 1, 2, 3, 1, 2, 3, 4]


def test_dequantize_known():  # :361-503
    assert DQ(np.array([0, 1, -1], np.int8), 1.0, 0).tolist() == [0, 1, -1]
    assert DQ(np.array([100, 101, 102], np.int8), 2.0, 100).tolist() == [0, 2, 4]
    assert DQ(np.array([128, 129, 127], np.uint8), 0.5, 128).tolist() == [0, 0.5, -0.5]
    x = np.array([[0, 0, 1], [10, 5, 4]], np.int8)
    assert DQ(x, [1, 2, 3], [0, 0, 0], axis=1).ravel().tolist() == [0, 0, 3, 10, 10, 12]
    x = np.array([[1, 2, 3], [4, 5, 6]], np.int8)
    assert DQ(x, [0.5, 2], [0, 0], axis=-1).ravel().tolist() == [0.5, 1, 1.5, 8, 10, 12]


def test_dequantize_random_and_roundtrip():  # :505-590
    rng = np.random.default_rng(7)
    q = rng.integers(-128, 128, (4, 8)).astype(np.int8)
    got = DQ(q, 1.5, -3)
    np.testing.assert_allclose(got, (q.astype(np.float64) + 3) * 1.5, atol=1e-4)
    x = rng.uniform(-5, 5, (4, 8)).astype(f32)
    back = DQ(Q(x, 0.1, 0), 0.1, 0)
    assert np.all(np.abs(back - x) <= 0.1 * 0.55)


# --- float64 restatements of each rounding step ------------------------------

def _round_f32(v64):
    return np.asarray(v64, np.float64).astype(f32)


def test_quantize_is_one_fma_rounded_to_even():
    """q = rint(x * (1/s) + zp) with the product-sum rounded once (FMA), ties to
    even: x * inv + zp is exact in float64 for these magnitudes, so a
    separate multiply-then-add or round-half-away rule fails on some element."""
    rng = np.random.default_rng(3)
    x = rng.normal(0, 30, 4096).astype(f32)
    x[:64] = np.arange(-32, 32, dtype=f32) + 0.5  # exact ties
    s = f32(0.37)
    inv = f32(1) / s
    for zp in (0, 5, -7):
        exact = x.astype(np.float64) * np.float64(inv) + zp   # exact (< 53 bits)
        want = np.clip(np.rint(_round_f32(exact)), -128, 127).astype(np.int8)
        assert np.array_equal(Q(x, s, zp), want)
    # a separate multiply-then-add rounds differently on some inputs
    sep = (x * inv).astype(f32) + f32(5)
    fused = _round_f32(x.astype(np.float64) * np.float64(inv) + 5)
    assert np.any(sep != fused)


def test_quantize_specials_saturate_to_qmin():
    x = np.array([np.nan, np.inf, -np.inf, 3e9, -3e9, 1e30], f32)
    assert Q(x, 1.0, 0).tolist() == [-128, -128, -128, -128, -128, -128]
    assert Q(x, 1.0, 0, out_dtype=np.uint8).tolist() == [0] * 6
    # finite values past the int8 range but below 2^31 clamp normally
    assert Q(np.array([1e6, -1e6], f32), 1.0, 0).tolist() == [127, -128]


def test_quantize_f16_input_widens_exactly():
    rng = np.random.default_rng(4)
    x = rng.normal(0, 20, 1000).astype(np.float16)
    assert np.array_equal(Q(x, 0.25, 3), Q(x.astype(f32), 0.25, 3))


@pytest.mark.parametrize("seg", [16, 37, 100])
def test_dequantize_body_fma_and_tail(seg):
    """Per segment: whole 16-blocks fma(q, s, f32(-zp*s)), the last seg % 16
    elements f32((q - zp) * s) (one rounding of an exact float64 product)."""
    rng = np.random.default_rng(seg)
    rows = 3
    q = rng.integers(-128, 128, (rows, seg)).astype(np.int8)
    s, zp = f32(0.1), 17
    got = DQ(q, np.full(rows, s), np.full(rows, zp), axis=-1)
    nzs = np.float64(_round_f32(-np.float64(zp) * np.float64(s)))
    body = _round_f32(q.astype(np.float64) * np.float64(s) + nzs)
    tail = _round_f32((q.astype(np.float64) - zp) * np.float64(s))
    cut = seg - seg % 16
    assert np.array_equal(got[:, :cut], body[:, :cut])
    assert np.array_equal(got[:, cut:], tail[:, cut:])
    # the two forms differ for some q at this scale, so the split is tested
    allq = np.arange(-128, 128, dtype=np.float64)
    assert np.any(_round_f32(allq * np.float64(s) + nzs) != _round_f32((allq - zp) * np.float64(s)))


def test_dequantize_per_tensor_segment_is_numel():
    q = np.random.default_rng(9).integers(-128, 128, (5, 7)).astype(np.int8)
    got = DQ(q, 0.1, 17).ravel()
    flat = DQ(q.ravel(), 0.1, 17)
    assert np.array_equal(got, flat)
    s = np.float64(f32(0.1))
    nzs = np.float64(_round_f32(-17 * s))
    qq = q.ravel().astype(np.float64)
    want = np.concatenate([_round_f32(qq[:32] * s + nzs), _round_f32((qq[32:] - 17) * s)])
    assert np.array_equal(got, want)


def test_dequantize_f16_output_is_rne_of_f32():
    q = np.arange(-128, 128, dtype=np.int8).reshape(16, 16)
    y32 = DQ(q, 0.0371, 3)
    y16 = DQ(q, 0.0371, 3, out_dtype=np.float16)
    assert np.array_equal(y16, y32.astype(np.float16))


def test_per_channel_middle_axis_indexing():
    """3-D per channel on axis 1: parameter of [i, j, k] is j."""
    q = np.random.default_rng(2).integers(-128, 128, (2, 3, 20)).astype(np.int8)
    sc = np.array([0.5, 0.25, 2.0], f32)
    zp = np.array([1, -2, 3])
    got = DQ(q, sc, zp, axis=1)
    want = (q.astype(np.float64) - zp[None, :, None]) * sc[None, :, None]
    assert np.array_equal(got, want.astype(f32))   # power-of-two scales: exact
    x = got
    assert np.array_equal(Q(x, sc, zp, axis=1), q)  # round trip through exact values


# --- the fp-activation int8 GEMM against the compiled reference --------------

ref_only = pytest.mark.skipif(oracle.ref_lib() is None, reason="oracle/_ref not built (no reference tree)")


def oracle_fp_a_gemm(a, b, *, trans_b, s_a, zp_a, s_b, zp_b, bias, act, alpha, beta, lo, hi, act_u8):
    """QuantizeLinear of A per token, then the int8 GEMM with a dequantizing
    destination in A's dtype: the composite the HIP front end runs."""
    M = a.shape[0]
    sa = np.broadcast_to(np.asarray(s_a, f32), (M,))
    za = np.broadcast_to(np.asarray(zp_a), (M,))
    aq = Q(a, sa, za, out_dtype=np.uint8 if act_u8 else np.int8, axis=-1)
    out = oracle.OUT_F16 if a.dtype == np.float16 else oracle.OUT_F32
    return oracle.gemm_i8(aq, b, trans_b=trans_b, out_kind=out, s_a=sa, zp_a=za.astype(np.int32),
                          s_b=s_b, zp_b=zp_b, bias=bias, act=act, act_alpha=alpha, act_beta=beta,
                          min_clip=lo, max_clip=hi)


def ref_fp_a_gemm(a, b, *, trans_b, s_a, zp_a, s_b, zp_b, bias, act, alpha, beta, lo, hi, act_u8):
    M, K = a.shape
    N = b.shape[0] if trans_b else b.shape[1]
    c = np.zeros((M, N), a.dtype)
    per_tok = np.ndim(s_a) > 0
    sa = np.ascontiguousarray(s_a, f32) if per_tok else None
    za = np.ascontiguousarray(zp_a, np.int32) if per_tok else None
    per_ch = np.ndim(s_b) > 0
    sb = np.ascontiguousarray(s_b, f32) if per_ch else None
    zb = np.ascontiguousarray(zp_b, np.int32) if per_ch else None
    oracle.ref_lib().ref_matmul_dq(
        a.ctypes.data, int(a.dtype == np.float16), b.ctypes.data,
        None if bias is None else bias.ctypes.data, c.ctypes.data,
        M, N, K, a.strides[0], b.strides[0], c.strides[0], int(trans_b), int(act_u8),
        None if sa is None else sa.ctypes.data, 1.0 if per_tok else float(s_a),
        None if za is None else za.ctypes.data, 0 if per_tok else int(zp_a),
        None if sb is None else sb.ctypes.data, 1.0 if per_ch else float(s_b),
        None if zb is None else zb.ctypes.data, 0 if per_ch else int(zp_b),
        act, alpha, beta, lo, hi)
    return c


@ref_only
@pytest.mark.parametrize("seed", range(12))
def test_fp_a_dq_gemm_matches_reference(seed):
    """Bit for bit: quantize A (per tensor / per token, s8 / u8), int8 GEMM with
    zero points, dequantize with bias, clip and every activation, f32 / f16."""
    rng = np.random.default_rng(seed)
    M, K, N = (int(v) for v in rng.integers(1, 60, 3))
    dt = np.float16 if seed & 1 else np.float32
    tb = bool(seed & 2)
    act_u8 = bool(seed & 4)
    a = rng.normal(0, 2, (M, K)).astype(dt)
    b = rng.integers(-128, 128, (N, K) if tb else (K, N)).astype(np.int8)
    if seed % 3 == 0:
        s_a, zp_a = f32(0.03), (130 if act_u8 else 3)
    else:
        s_a = rng.uniform(0.01, 0.05, M).astype(f32)
        zp_a = rng.integers(100, 150, M) if act_u8 else rng.integers(-5, 5, M)
    s_b = rng.uniform(0.002, 0.02, N).astype(f32) if seed & 8 else f32(0.01)
    zp_b = rng.integers(-3, 3, N) if seed & 8 else 0
    bias = rng.normal(0, 1, N).astype(dt) if seed % 4 != 1 else None
    act = seed % 10
    lo, hi = (-4.0, 5.0) if seed % 5 == 0 else (-np.inf, np.inf)
    kw = dict(trans_b=tb, s_a=s_a, zp_a=zp_a, s_b=s_b, zp_b=zp_b, bias=bias, act=act,
              alpha=0.1, beta=0.7, lo=lo, hi=hi, act_u8=act_u8)
    got = oracle_fp_a_gemm(a, b, **kw)
    want = ref_fp_a_gemm(a, b, **kw)
    np.testing.assert_array_equal(got.view(np.uint16 if dt == np.float16 else np.uint32),
                                  want.view(np.uint16 if dt == np.float16 else np.uint32))
