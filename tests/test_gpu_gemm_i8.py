"""int8 GEMM / GEMV on the GPU through the C ABI (nnops_hip_gemm_i8), bit-exact
against the CPU oracle and the reference's golden vectors."""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import pytest

import oracle
import datagen as dg
import nnops_amd as na
from golden.gen_golden import build_i8_case, OUTK, ODT
from gpu_util import dev, pitched, host, announce, oracle_rows

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden.json")))
TORCH_ODT = None


def torch_dt(np_dt):
    import torch
    return {np.int32: torch.int32, np.int8: torch.int8, np.uint8: torch.uint8}[np_dt]


def scal_or_dev(x):
    return dev(x) if isinstance(x, np.ndarray) else x.item() if hasattr(x, "item") else x


def run_gpu(a, b, out_kind, *, trans_b, bias=None, s_a=1.0, zp_a=0, s_b=1.0, zp_b=0, s_out=1.0,
            zp_out=0, relu=False, round_even=False, trans_a=False, lda=None, ldc=None, c_init=None,
            float_ep=False, act=None, add_to=False, residual_pre=False, s_out_rows=None,
            zp_out_rows=None, c_dev=None):
    import torch
    odt = {0: np.int32, 1: np.int8, 2: np.uint8}[out_kind]
    M = a.shape[1] if trans_a else a.shape[0]
    N = b.shape[0] if trans_b else b.shape[1]
    da = pitched(a, lda) if lda else dev(a)
    db = dev(b)
    if c_dev is not None:
        dc = c_dev
    else:
        if c_init is None:
            c_init = np.zeros((M, N), odt)
        dc = pitched(c_init, ldc) if ldc else dev(c_init)
    kw = dict(trans_a=trans_a, trans_b=trans_b, out_kind=out_kind, bias=None if bias is None else dev(bias),
              s_a=scal_or_dev(s_a), zp_a=scal_or_dev(zp_a), s_b=scal_or_dev(s_b), zp_b=scal_or_dev(zp_b),
              s_out=float(s_out), zp_out=int(zp_out), round_even=round_even, float_ep=float_ep,
              act=act if act is not None else (na.ACT_RELU if relu else na.ACT_NONE),
              add_to=add_to, residual_pre=residual_pre,
              s_out_rows=None if s_out_rows is None else dev(s_out_rows),
              zp_out_rows=None if zp_out_rows is None else dev(zp_out_rows))
    na.gemm_i8(da, db, dc, **kw)
    torch.cuda.synchronize()
    return host(dc)


@pytest.mark.parametrize("entry", GOLD["i8"], ids=[e["case"]["name"] for e in GOLD["i8"]])
def test_golden_cases_bit_exact(entry):
    c = entry["case"]
    announce(f"golden {c['name']}")
    ops = build_i8_case(c)
    got = run_gpu(ops["a"], ops["b"], OUTK[c["out"]], trans_b=c["trans_b"], bias=ops["bias"],
                  s_a=ops["s_a"], zp_a=ops["zp_a"], s_b=ops["s_b"], zp_b=ops["zp_b"],
                  s_out=c.get("s_out", 1.0), zp_out=c.get("zp_out", 0), relu=c.get("relu", False),
                  lda=c.get("lda"))
    assert hashlib.sha256(np.ascontiguousarray(got).tobytes()).hexdigest() == entry["out"]["sha256"]


SHAPES = [
    # (M, K, N): GEMV (M<=16), small-tile, mid-tile, large-tile routes, ragged
    (1, 64, 16), (1, 4096, 1000), (3, 100, 37), (16, 512, 130), (17, 96, 65),
    (33, 208, 70), (64, 4096, 64), (100, 1000, 333), (130, 64, 1030), (300, 512, 257),
    (1024, 256, 1024), (1100, 160, 1050),
    # ring-kernel tile shapes, K splits and the fused / partial output modes
    (96, 512, 512), (200, 1024, 256), (333, 2048, 512), (1024, 512, 4096),
    # column GEMV on a [K,N] B (16- and 4-column lane groups, K splits)
    (2, 4096, 1008), (5, 256, 100), (12, 1024, 2048), (16, 512, 4096),
    (1, 1040, 8192), (2, 1024, 8256), (7, 512, 8192),
    # row GEMV with two rows per wave (M = 3..4), LDS-staged skinny GEMM
    # (4 < M <= 16) with a ragged last group of rows and a K tail past 4 KiB
    (3, 512, 130), (4, 4096, 1000), (8, 5120, 77), (16, 1088, 4099),
    # [K,N] B staged by the 16-byte tiled transpose: partial 256-row and
    # 64-column tiles, and K % 16 != 0 (the zero-filled rows K..Kp-1)
    (64, 992, 1040), (130, 1040, 1008), (48, 1000, 1040),
    # [K,N] B read in place by the ring (transposed LDS reads): N past the last
    # 16-byte chunk, 64-byte stages (K % 128 != 0), 64 x 64 tiles of small grids
    (200, 1024, 252), (96, 640, 1000), (64, 256, 200), (128, 1024, 1024),
]


@pytest.mark.parametrize("M,K,N", SHAPES)
@pytest.mark.parametrize("trans_b", [True, False])
def test_random_shapes_s32_and_s8(M, K, N, trans_b):
    announce(f"random {M}x{K}x{N} trans_b={trans_b}")
    seed = M * 7 + K * 3 + N + int(trans_b)
    a = dg.ints(seed, (M, K), -128, 127)
    b = dg.ints(seed + 1, (N, K) if trans_b else (K, N), -128, 127)
    bias = dg.ints(seed + 2, (N,), -20000, 20000, np.int32)
    got = run_gpu(a, b, na.OUT_S32, trans_b=trans_b, bias=bias)
    want = oracle.gemm_i8(a, b, trans_b=trans_b, bias=bias)
    np.testing.assert_array_equal(got, want)
    sb = dg.uniform(seed + 3, (N,), 0.001, 0.01)
    s_out = 0.02 * 0.0055 * 73 * np.sqrt(K) * 75 / 60
    got = run_gpu(a, b, na.OUT_S8, trans_b=trans_b, bias=bias, s_a=0.02, s_b=sb, s_out=s_out, relu=True)
    want = oracle.gemm_i8(a, b, trans_b=trans_b, bias=bias, out_kind=oracle.OUT_S8, s_a=0.02, s_b=sb,
                          s_out=s_out, act=oracle.ACT_RELU)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("M,K,N", [(5, 77, 9), (40, 300, 33), (200, 130, 90), (300, 640, 256)])
def test_u8_zero_points_trans_a_round_even(M, K, N):
    announce(f"u8/zp/trans_a {M}x{K}x{N}")
    seed = 77 + M
    a = dg.ints(seed, (K, M), 0, 255, np.uint8)  # [K, M]: trans_a
    b = dg.ints(seed + 1, (K, N), -128, 127)
    zpa = dg.ints(seed + 2, (M,), 100, 150, np.int32)
    zpb = dg.ints(seed + 3, (N,), -3, 3, np.int32)
    sa = dg.uniform(seed + 4, (M,), 0.01, 0.05)
    for out_kind, zp_out in ((na.OUT_S32, 0), (na.OUT_S8, -7), (na.OUT_U8, 128)):
        for even in (False, True):
            got = run_gpu(a, b, out_kind, trans_a=True, trans_b=False, s_a=sa, zp_a=zpa, zp_b=zpb,
                          s_out=256.0, zp_out=zp_out, round_even=even)
            want = oracle.gemm_i8(a, b, trans_a=True, out_kind=out_kind, s_a=sa, zp_a=zpa, zp_b=zpb,
                                  s_out=256.0, zp_out=zp_out, round_even=even)
            np.testing.assert_array_equal(got, want)


def test_per_row_output_table():
    announce("per-row requant table")
    M, K, N = 50, 256, 70
    a = dg.act_s8(31, (M, K))
    b = dg.ints(32, (N, K), -127, 127)
    so = dg.uniform(33, (M,), 0.5, 3.0)
    zo = dg.ints(34, (M,), -10, 10, np.int32)
    got = run_gpu(a, b, na.OUT_S8, trans_b=True, s_a=0.02, s_b=0.005, s_out_rows=so, zp_out_rows=zo)
    want = oracle.gemm_i8(a, b, trans_b=True, out_kind=oracle.OUT_S8, s_a=0.02, s_b=0.005,
                          s_out_rows=so, zp_out_rows=zo)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("residual_pre", [False, True])
@pytest.mark.parametrize("M", [7, 333])
def test_float_epilogue_add_to_gelu_pitched(M, residual_pre):
    """Config 5's composite (s8 add_to + GELU via f32 + requant) on pitched A
    and C: no nnops route exists (parity unpinned vs nnops); bit-exact vs the
    oracle's definition of it."""
    announce(f"float epilogue M={M} pre={residual_pre}")
    K, N = 1024, 520
    a = dg.act_s8(41 + M, (M, K))
    b = dg.ints(42, (K, N), -127, 127)
    sb = dg.uniform(43, (N,), 0.001, 0.01)
    bias = dg.ints(44, (N,), -5000, 5000, np.int32)
    c0 = dg.ints(45, (M, N), -128, 127)
    s_out = 0.05 * 40
    got = run_gpu(a, b, na.OUT_S8, trans_b=False, bias=bias, s_a=0.02, s_b=sb, s_out=s_out, zp_out=2,
                  lda=K + 64, ldc=N + 64, c_init=c0, float_ep=True, act=na.ACT_GELU, add_to=True,
                  residual_pre=residual_pre)
    want = oracle.gemm_i8(a, b, bias=bias, out_kind=oracle.OUT_S8, s_a=0.02, s_b=sb, s_out=s_out,
                          zp_out=2, float_ep=True, act=oracle.ACT_GELU, add_to=True,
                          residual_pre=residual_pre, c=c0.copy())
    assert np.unique(want).size > 50  # not a saturated comparison
    np.testing.assert_array_equal(got, want)


def test_trans_a_pitched_partial_transpose_segments():
    """A stored [K][M] with a 16-byte pitch wider than M: the tiled transpose
    reads the rows' last, partial 16-byte pieces byte by byte."""
    announce("trans_a pitched")
    M, K, N = 40, 300, 64
    at = dg.ints(71, (K, M), -127, 127)
    b = dg.ints(72, (N, K), -127, 127)
    got = run_gpu(at, b, na.OUT_S32, trans_b=True, trans_a=True, lda=48)
    want = oracle.gemm_i8(at, b, trans_b=True, trans_a=True)
    np.testing.assert_array_equal(got, want)


def test_determinism_repeated_runs():
    announce("determinism")
    M, K, N = 300, 2048, 700
    a = dg.ints(51, (M, K), -127, 127)
    b = dg.ints(52, (N, K), -127, 127)
    r1 = run_gpu(a, b, na.OUT_S32, trans_b=True)
    r2 = run_gpu(a, b, na.OUT_S32, trans_b=True)
    np.testing.assert_array_equal(r1, r2)


def test_timed_launch_same_result_and_positive_time():
    """A launch armed with nnops_hip_time_next_launch (events on its dispatch
    packet) computes the same bits as an unarmed one, and its events measure
    a positive kernel time."""
    import ctypes as C
    import torch
    announce("timed launch")
    M, K, N = 256, 1024, 512
    a = dg.act_s8(61, (M, K))
    b = dg.ints(62, (N, K), -127, 127)
    want = oracle.gemm_i8(a, b, trans_b=True, out_kind=oracle.OUT_S32)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    e1.record()
    torch.cuda.synchronize()
    assert na.lib().nnops_hip_time_next_launch(C.c_void_p(e0.cuda_event), C.c_void_p(e1.cuda_event)) == na.OK
    got = run_gpu(a, b, na.OUT_S32, trans_b=True)
    assert e0.elapsed_time(e1) > 0.0
    np.testing.assert_array_equal(got, want)
    # one-shot: the next call runs unarmed and still matches
    np.testing.assert_array_equal(run_gpu(a, b, na.OUT_S32, trans_b=True), want)


@pytest.mark.parametrize("M", [1, 4, 16])
def test_config3_full_gemv(M):
    """BASELINE config 3 at full size (K=4096, N=11008), s32 and s8."""
    announce(f"config3 M={M}")
    K, N = 4096, 11008
    a = dg.ints(61 + M, (M, K), -127, 127)
    b = dg.ints(62, (K, N), -127, 127)
    got = run_gpu(a, b, na.OUT_S32, trans_b=False)
    want = oracle.gemm_i8(a, b)
    np.testing.assert_array_equal(got, want)
    sb = dg.uniform(63, (N,), 0.001, 0.01)
    bt = np.ascontiguousarray(b.T)
    got = run_gpu(a, bt, na.OUT_S8, trans_b=True, s_a=0.02, s_b=sb, s_out=0.05)
    want = oracle.gemm_i8(a, bt, trans_b=True, out_kind=oracle.OUT_S8, s_a=0.02, s_b=sb, s_out=0.05)
    np.testing.assert_array_equal(got, want)


def test_config2_full_every_row():
    """BASELINE config 2 at full size: M=N=K=4096, s8 out with per-channel
    scales, bias and Relu; every output compared bit for bit. The expected
    tile comes from nnops' own CPU MatMul (oracle/_ref/libnnops_cpu.so, whose
    outputs the oracle matches bit for bit) where this host runs it, else
    from the oracle in row bands over the host's cores."""
    announce("config2 full, every row")
    M = N = K = 4096
    a = dg.act_s8(71, (M, K))
    w = dg.ints(72, (N, K), -127, 127)
    sb = dg.uniform(73, (N,), 0.001, 0.01)
    bias = dg.ints(74, (N,), -5000, 5000, np.int32)
    got = run_gpu(a, w, na.OUT_S8, trans_b=True, bias=bias, s_a=0.02, s_b=sb, s_out=0.05, relu=True)
    cpu = oracle.cpu_lib()
    if cpu is not None:
        want = np.zeros((M, N), np.int8)
        rc = cpu.ref_cpu_matmul_s8(a.ctypes.data, w.ctypes.data, bias.ctypes.data, want.ctypes.data, M, N, K,
                                   0.02, sb.ctypes.data, 0.05, 0, 1, 16)
        assert rc == 0, rc
        # the two checkers agree on bands spread over the tiles
        for r0 in (0, 1000, 4080):
            np.testing.assert_array_equal(
                want[r0:r0 + 16], oracle.gemm_i8(a, w, trans_b=True, bias=bias, out_kind=oracle.OUT_S8, s_a=0.02,
                                                 s_b=sb, s_out=0.05, act=oracle.ACT_RELU, rows=(r0, r0 + 16))[r0:r0 + 16])
    else:
        want = oracle_rows(lambda r0, r1: oracle.gemm_i8(
            a, w, trans_b=True, bias=bias, out_kind=oracle.OUT_S8, s_a=0.02, s_b=sb, s_out=0.05,
            act=oracle.ACT_RELU, rows=(r0, r1))[r0:r1], M)
    np.testing.assert_array_equal(got, want)
    assert got.min() >= 0 and np.unique(got).size > 100


@pytest.mark.parametrize("M", [1, 3, 16])
def test_kn_gemv_weight_zero_point_and_tables(M):
    """[K,N] weights consumed in place: weight zero points (row sums of A),
    per-column scales, per-row output tables."""
    announce(f"[K,N] GEMV zp_b M={M}")
    K, N = 2048, 1536
    a = dg.act_s8(90 + M, (M, K))
    b = dg.ints(91, (K, N), -127, 127)
    zpb = dg.ints(92, (N,), -4, 4, np.int32)
    sb = dg.uniform(93, (N,), 0.005, 0.02)
    so = dg.uniform(94, (M,), 0.5, 2.0)
    bias = dg.ints(95, (N,), -5000, 5000, np.int32)
    got = run_gpu(a, b, na.OUT_S8, trans_b=False, bias=bias, s_a=0.02, s_b=sb, zp_b=zpb, s_out_rows=so, relu=True)
    want = oracle.gemm_i8(a, b, bias=bias, out_kind=oracle.OUT_S8, s_a=0.02, s_b=sb, zp_b=zpb,
                          s_out_rows=so, act=oracle.ACT_RELU)
    assert np.unique(want).size > 50
    np.testing.assert_array_equal(got, want)
    got = run_gpu(a, b, na.OUT_S32, trans_b=False, zp_b=zpb)
    np.testing.assert_array_equal(got, oracle.gemm_i8(a, b, zp_b=zpb))


def test_kn_split_meeting_reuses_one_workspace():
    """The [K,N] MFMA GEMV (3 <= M <= 16) meets its K splits inside the
    launch through completion flags in the workspace (the column GEMV at
    M <= 2, which sums its splits in a second launch, rides along): a workspace filled with 0xff bytes
    (flag words that are not the launch's epoch), then the same workspace
    again (the flags left cleared), then a smaller call over it, each bit for
    bit against the oracle, s32 and s8 destinations."""
    import torch
    ws = torch.full((32 << 20,), 0xff, dtype=torch.uint8, device="cuda")
    for M, K, N, out in [(16, 4096, 2048, "s32"), (16, 4096, 2048, "s8"), (5, 1024, 1000, "s32"),
                         (12, 2048, 4096, "s8"), (1, 4096, 11008, "s32"), (2, 1024, 8256, "s8"),
                         (1, 2048, 1040, "s8")]:
        announce(f"[K,N] split meeting {M}x{K}x{N} {out}")
        a = dg.act_s8(700 + M, (M, K))
        b = dg.ints(701 + N, (K, N), -127, 127)
        sb = dg.uniform(702, (N,), 0.002, 0.01)
        bias = dg.ints(703, (N,), -3000, 3000, np.int32)
        kind = na.OUT_S32 if out == "s32" else na.OUT_S8
        c = torch.zeros((M, N), dtype=torch.int32 if out == "s32" else torch.int8, device="cuda")
        for rep in range(2):
            c.zero_()
            na.gemm_i8(dev(a), dev(b), c, trans_b=False, out_kind=kind, bias=dev(bias), s_a=0.02, s_b=dev(sb),
                       s_out=0.05, act=na.ACT_RELU, workspace=ws)
            torch.cuda.synchronize()
            want = oracle.gemm_i8(a, b, bias=bias, out_kind=oracle.OUT_S32 if out == "s32" else oracle.OUT_S8,
                                  s_a=0.02, s_b=sb, s_out=0.05, act=oracle.ACT_RELU)
            np.testing.assert_array_equal(host(c), want, err_msg=f"call {rep}")


@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("s_out", [0.05, 2.0])
def test_config5_full_workload_every_row(trans_b, s_out):
    """BASELINE config 5 at its real workload: M=333, K=14336, N=4096, A row
    pitch 14400 B, C row pitch 4160 B (sentinel-filled padding), s8 add_to
    residual into a pre-filled C, GELU through the f32 epilogue, requant.
    s_out 0.05 is the config's literal scale (mostly saturated outputs);
    2.0 keeps most outputs inside (-128, 127). The weight is the MatMul's
    [K,N] (trans_b False) or the Linear's [N,K]. Every row is compared bit
    for bit with the oracle; the padding must be untouched."""
    announce(f"config5 full trans_b={trans_b} s_out={s_out}")
    M, K, N, LDA, LDC = 333, 14336, 4096, 14400, 4160
    a = dg.act_s8(501, (M, K))
    w = dg.ints(502, (K, N), -127, 127)
    if trans_b:
        w = np.ascontiguousarray(w.T)
    sb = dg.uniform(503, (N,), 0.001, 0.01)
    bias = dg.ints(504, (N,), -5000, 5000, np.int32)
    c0 = dg.ints(505, (M, N), -128, 127)
    import torch
    dc = pitched(c0, LDC)
    got = run_gpu(a, w, na.OUT_S8, trans_b=trans_b, bias=bias, s_a=0.02, s_b=sb, s_out=s_out, lda=LDA,
                  c_init=None, ldc=None, float_ep=True, act=na.ACT_GELU, add_to=True, residual_pre=False,
                  c_dev=dc)
    pad = host(dc.as_strided((M, LDC - N), (LDC, 1), dc.storage_offset() + N))
    assert np.all(pad == 0x5A), "C padding written"
    want = oracle_rows(lambda r0, r1: oracle.gemm_i8(
        a, w, trans_b=trans_b, bias=bias, out_kind=oracle.OUT_S8, s_a=0.02, s_b=sb, s_out=s_out, float_ep=True,
        act=oracle.ACT_GELU, add_to=True, residual_pre=False, c=c0.copy(), rows=(r0, r1))[r0:r1], M, band=8)
    np.testing.assert_array_equal(got, want)
    if s_out == 2.0:
        assert np.mean((got > -128) & (got < 127)) > 0.5
