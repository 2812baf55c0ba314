"""ctypes front end of the CPU oracle (test infrastructure only).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this package, always as the checker and never as the thing measured or
shipped. ``liboracle.so`` is built from ``oracle.c`` by ``make -C oracle``;
``_ref/libnnops_ref.so`` (the reference's own oracles, built from the nnops
sources by ``make -C oracle ref``) is optional and only present where the
reference tree was available at build time.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))

OUT_S32, OUT_S8, OUT_U8, OUT_F32, OUT_F16 = 0, 1, 2, 3, 4
(ACT_NONE, ACT_RELU, ACT_GELU, ACT_SIGMOID, ACT_TANH, ACT_LEAKY_RELU, ACT_SILU, ACT_HARDSWISH, ACT_ELU,
 ACT_RELU6) = range(10)


class GemmI8(C.Structure):
    _fields_ = [
        ("a", C.c_void_p), ("b", C.c_void_p), ("bias", C.c_void_p), ("c", C.c_void_p),
        ("m", C.c_int64), ("n", C.c_int64), ("k", C.c_int64),
        ("lda", C.c_int64), ("ldb", C.c_int64), ("ldc", C.c_int64),
        ("trans_a", C.c_int32), ("trans_b", C.c_int32), ("a_u8", C.c_int32),
        ("s_a", C.c_void_p), ("s_a_scalar", C.c_float), ("zp_a", C.c_void_p), ("zp_a_scalar", C.c_int32),
        ("s_b", C.c_void_p), ("s_b_scalar", C.c_float), ("zp_b", C.c_void_p), ("zp_b_scalar", C.c_int32),
        ("s_out_rows", C.c_void_p), ("zp_out_rows", C.c_void_p), ("s_out", C.c_float), ("zp_out", C.c_int32),
        ("out_kind", C.c_int32), ("act", C.c_int32), ("round_even", C.c_int32),
        ("float_ep", C.c_int32), ("min_clip", C.c_float), ("max_clip", C.c_float),
        ("add_to", C.c_int32), ("residual_pre", C.c_int32),
        ("m_begin", C.c_int64), ("m_end", C.c_int64),
        ("act_alpha", C.c_float), ("act_beta", C.c_float),
    ]


class GemmQ41(C.Structure):
    _fields_ = [
        ("a", C.c_void_p), ("b", C.c_void_p), ("c", C.c_void_p),
        ("m", C.c_int64), ("n", C.c_int64), ("k", C.c_int64),
        ("lda", C.c_int64), ("ldc", C.c_int64), ("ldb_bytes", C.c_int64),
        ("trans_b", C.c_int32), ("a_f16", C.c_int32), ("c_f16", C.c_int32),
        ("w_round_f16", C.c_int32), ("acc_f64", C.c_int32),
        ("m_begin", C.c_int64), ("m_end", C.c_int64),
    ]


class FpOut(C.Structure):
    _fields_ = [
        ("src", C.c_void_p), ("ld_src", C.c_int64), ("out", C.c_void_p), ("ld_out", C.c_int64),
        ("rows", C.c_int64), ("n", C.c_int64), ("out_f16", C.c_int32), ("bias", C.c_void_p),
        ("act", C.c_int32), ("act_alpha", C.c_float), ("act_beta", C.c_float),
        ("min_clip", C.c_float), ("max_clip", C.c_float),
        ("add_to", C.c_int32), ("residual_pre", C.c_int32), ("gated", C.c_int32), ("gate_act", C.c_int32),
        ("gate_alpha", C.c_float), ("gate_beta", C.c_float), ("gate_limit", C.c_float),
        ("matmul_order", C.c_int32), ("alpha", C.c_float), ("beta", C.c_float),
    ]


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle not built: {path} (run `make -C oracle`)")
        _lib = C.CDLL(path)
        _lib.orc_gemm_i8.argtypes = [C.POINTER(GemmI8)]
        _lib.orc_gemm_q4_1.argtypes = [C.POINTER(GemmQ41)]
        _lib.orc_requant.argtypes = [C.c_int32, C.c_float, C.c_int32, C.c_int32, C.c_int32]
        _lib.orc_requant.restype = C.c_int32
        _lib.orc_requant_scale.argtypes = [C.c_float] * 3
        _lib.orc_requant_scale.restype = C.c_float
        _lib.orc_tanhf.argtypes = [C.c_float]
        _lib.orc_tanhf.restype = C.c_float
        _lib.orc_gelu_tanh.argtypes = [C.c_float]
        _lib.orc_gelu_tanh.restype = C.c_float
        _lib.orc_markstein_mismatches.argtypes = [C.c_float, C.c_uint32, C.c_uint32, C.c_uint32, C.c_int32]
        _lib.orc_markstein_mismatches.restype = C.c_int64
        _lib.orc_f32_to_f16.argtypes = [C.c_float]
        _lib.orc_f32_to_f16.restype = C.c_uint16
        _lib.orc_f16_to_f32.argtypes = [C.c_uint16]
        _lib.orc_f16_to_f32.restype = C.c_float
        _lib.orc_fp_out_pass.argtypes = [C.POINTER(FpOut)]
        _lib.orc_q4_1_decode.argtypes = [C.c_void_p, C.c_int64, C.c_void_p]
        _lib.orc_q4_1_quantize.argtypes = [C.c_void_p, C.c_int64, C.c_void_p]
        _lib.orc_quantize_linear.argtypes = [C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_int64,
                                             C.c_void_p, C.c_void_p, C.c_int64, C.c_int64]
        _lib.orc_dequantize_linear.argtypes = [C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_int64,
                                               C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int64]
    return _lib


def ref_lib():
    """The reference's own oracles, or None where they were not built."""
    global _ref
    if _ref is None:
        path = os.path.join(_HERE, "_ref", "libnnops_ref.so")
        if not os.path.exists(path):
            return None
        _ref = C.CDLL(path)
        _ref.ref_matmul_int8.argtypes = [
            C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
            C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64,
            C.c_int, C.c_int,
            C.c_void_p, C.c_float, C.c_void_p, C.c_int32,
            C.c_void_p, C.c_float, C.c_void_p, C.c_int32,
            C.c_float, C.c_int32, C.c_int, C.c_int]
        for nm in ("ref_requant_s8", "ref_requant_u8"):
            getattr(_ref, nm).argtypes = [C.c_int32, C.c_float, C.c_int32]
            getattr(_ref, nm).restype = C.c_int32
        _ref.ref_requant_scale.argtypes = [C.c_float] * 3
        _ref.ref_requant_scale.restype = C.c_float
        _ref.ref_q4_1_quantize.argtypes = [C.c_void_p, C.c_int64, C.c_void_p]
        _ref.ref_q4_1_decode.argtypes = [C.c_void_p, C.c_int64, C.c_void_p]
        _ref.ref_matmul_dq.argtypes = [
            C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
            C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64,
            C.c_int, C.c_int,
            C.c_void_p, C.c_float, C.c_void_p, C.c_int32,
            C.c_void_p, C.c_float, C.c_void_p, C.c_int32,
            C.c_int, C.c_float, C.c_float, C.c_float, C.c_float]
        _ref.ref_gelu.argtypes = [C.c_float]
        _ref.ref_gelu.restype = C.c_float
        _ref.ref_f32_to_f16.argtypes = [C.c_float]
        _ref.ref_f32_to_f16.restype = C.c_uint16
        _ref.ref_f16_to_f32.argtypes = [C.c_uint16]
        _ref.ref_f16_to_f32.restype = C.c_float
    return _ref


_cpu = None


def cpu_lib():
    """nnops' own CPU MatMul (oracle/_ref/libnnops_cpu.so: its AVX-512-VNNI
    int8 route compiled from the reference sources), or None where it was not
    built or this host lacks AVX-512 VNNI/VL/BW (loading it would then fault
    on the first vector instruction)."""
    global _cpu
    if _cpu is None:
        path = os.path.join(_HERE, "_ref", "libnnops_cpu.so")
        if not os.path.exists(path) or not host_has_avx512_vnni():
            return None
        _cpu = C.CDLL(path)
        _cpu.ref_cpu_matmul_s8.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64,
                                           C.c_int64, C.c_float, C.c_void_p, C.c_float, C.c_int32, C.c_int,
                                           C.c_int]
        _cpu.ref_cpu_matmul_s8.restype = C.c_int
        _cpu.ref_cpu_matmul_i8.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64,
                                           C.c_int64, C.c_int, C.c_int, C.c_float, C.c_void_p, C.c_float,
                                           C.c_int32, C.c_int, C.c_int]
        _cpu.ref_cpu_matmul_i8.restype = C.c_int
        _cpu.ref_cpu_matmul_q4_1.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int64,
                                             C.c_int, C.c_int]
        _cpu.ref_cpu_matmul_q4_1.restype = C.c_int
        _cpu.ref_cpu_matmul_q4_1_ep.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                                C.c_int64, C.c_int64, C.c_int64, C.c_int, C.c_float, C.c_float,
                                                C.c_int, C.c_int, C.c_float, C.c_float, C.c_float, C.c_float,
                                                C.c_int]
        _cpu.ref_cpu_matmul_q4_1_ep.restype = C.c_int
        _cpu.ref_cpu_matmul_fp.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int64,
                                           C.c_int, C.c_int, C.c_int]
        _cpu.ref_cpu_matmul_fp.restype = C.c_int
        _cpu.ref_cpu_linear_fp.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64,
                                           C.c_int64, C.c_int64, C.c_int, C.c_float, C.c_float, C.c_float,
                                           C.c_float, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float,
                                           C.c_float, C.c_int]
        _cpu.ref_cpu_linear_fp.restype = C.c_int
        _cpu.ref_cpu_linear_q4_1.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64,
                                             C.c_int64, C.c_int64, C.c_int, C.c_float, C.c_float, C.c_float,
                                             C.c_float, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float,
                                             C.c_float, C.c_int]
        _cpu.ref_cpu_linear_q4_1.restype = C.c_int
        _cpu.ref_cpu_prepack_i8.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_int, C.c_int, C.c_void_p,
                                            C.c_int]
        _cpu.ref_cpu_prepack_i8.restype = C.c_void_p
        _cpu.ref_cpu_packed_free.argtypes = [C.c_void_p]
        _cpu.ref_cpu_packed_free.restype = None
        _cpu.ref_cpu_matmul_i8_packed.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64,
                                                  C.c_int64, C.c_int64, C.c_float, C.c_void_p, C.c_float,
                                                  C.c_int32, C.c_int, C.c_int]
        _cpu.ref_cpu_matmul_i8_packed.restype = C.c_int
        _cpu.ref_cpu_matmul_dq_f16.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                               C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int,
                                               C.c_int]
        _cpu.ref_cpu_matmul_dq_f16.restype = C.c_int
        _cpu.ref_cpu_qdq_f16.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64,
                                         C.c_int, C.c_int]
        _cpu.ref_cpu_qdq_f16.restype = C.c_int
    return _cpu


def host_has_avx512_vnni():
    try:
        flags = set()
        for line in open("/proc/cpuinfo"):
            if line.startswith("flags"):
                flags = set(line.split(":", 1)[1].split())
                break
    except OSError:
        return False
    return {"avx512f", "avx512_vnni", "avx512vl", "avx512bw", "avx2", "fma", "f16c"} <= flags


def _p(x):
    return None if x is None else x.ctypes.data


def gemm_i8(a, b, *, trans_b=False, trans_a=False, bias=None, out_kind=OUT_S32,
            s_a=1.0, zp_a=0, s_b=1.0, zp_b=0, s_out=1.0, zp_out=0,
            s_out_rows=None, zp_out_rows=None, act=ACT_NONE, round_even=False,
            float_ep=False, min_clip=-np.inf, max_clip=np.inf, add_to=False,
            residual_pre=False, c=None, rows=None, m=None, n=None, k=None, act_alpha=0.0, act_beta=1.0):
    """Run the oracle on numpy operands.

    ``a``: int8/uint8 2-D array ([M,K], or [K,M] with trans_a); its row stride is
    taken from the array's strides so a pitched view (a slice of a wider buffer)
    is honoured. ``b``: int8 [K,N] or [N,K] with trans_b. Scales/zero points may
    be scalars or 1-D arrays (per row of A / per column of the output). ``c``
    (optional) is the destination, read first when ``add_to``. ``rows``:
    (begin, end) to compute only those output rows. Returns ``c``.
    """
    a_u8 = a.dtype == np.uint8
    assert a.dtype in (np.int8, np.uint8) and b.dtype == np.int8
    assert a.strides[1] == 1 and b.strides[1] == 1
    M = a.shape[1] if trans_a else a.shape[0]
    K = a.shape[0] if trans_a else a.shape[1]
    N = b.shape[0] if trans_b else b.shape[1]
    odt = {OUT_S32: np.int32, OUT_S8: np.int8, OUT_U8: np.uint8, OUT_F32: np.float32,
           OUT_F16: np.float16}[out_kind]
    if c is None:
        c = np.zeros((M, N), dtype=odt)
    assert c.dtype == odt and c.strides[1] == c.itemsize
    keep = []

    def arr(x, dt):
        if x is None or np.isscalar(x):
            return None
        x = np.ascontiguousarray(x, dtype=dt)
        keep.append(x)
        return x

    s_a_arr, zp_a_arr = arr(s_a, np.float32), arr(zp_a, np.int32)
    s_b_arr, zp_b_arr = arr(s_b, np.float32), arr(zp_b, np.int32)
    so_arr, zo_arr = arr(s_out_rows, np.float32), arr(zp_out_rows, np.int32)
    bias_arr = None
    if bias is not None:
        bias_arr = arr(bias, {OUT_F32: np.float32, OUT_F16: np.float16}.get(out_kind, np.int32))
    p = GemmI8()
    p.a, p.b, p.c = a.ctypes.data, b.ctypes.data, c.ctypes.data
    p.bias = _p(bias_arr)
    p.m, p.n, p.k = M, N, K
    p.lda, p.ldb, p.ldc = a.strides[0], b.strides[0], c.strides[0] // c.itemsize
    p.trans_a, p.trans_b, p.a_u8 = int(trans_a), int(trans_b), int(a_u8)
    p.s_a, p.s_a_scalar = _p(s_a_arr), float(s_a) if s_a_arr is None else 1.0
    p.zp_a, p.zp_a_scalar = _p(zp_a_arr), int(zp_a) if zp_a_arr is None else 0
    p.s_b, p.s_b_scalar = _p(s_b_arr), float(s_b) if s_b_arr is None else 1.0
    p.zp_b, p.zp_b_scalar = _p(zp_b_arr), int(zp_b) if zp_b_arr is None else 0
    p.s_out_rows, p.zp_out_rows = _p(so_arr), _p(zo_arr)
    p.s_out, p.zp_out = float(s_out), int(zp_out)
    p.out_kind, p.act, p.round_even = out_kind, act, int(round_even)
    p.float_ep, p.min_clip, p.max_clip = int(float_ep), float(min_clip), float(max_clip)
    p.add_to, p.residual_pre = int(add_to), int(residual_pre)
    p.m_begin, p.m_end = (rows if rows is not None else (0, 0))
    p.act_alpha, p.act_beta = float(act_alpha), float(act_beta)
    lib().orc_gemm_i8(C.byref(p))
    return c


def gemm_q4_1(a, blocks, n, *, trans_b=True, ldb_bytes=None, c_f16=False,
              w_round_f16=False, acc_f64=True, rows=None):
    """f32 dequant GEMM over Q4_1 weights. ``a``: f16 or f32 [M,K] (row stride
    from its strides); ``blocks``: uint8 2-D array of rows of 20-byte blocks
    ([N][K/32] with trans_b, else [K][N/32])."""
    assert a.dtype in (np.float16, np.float32) and a.strides[1] == a.itemsize
    M, K = a.shape
    c = np.zeros((M, n), dtype=np.float16 if c_f16 else np.float32)
    p = GemmQ41()
    p.a, p.b, p.c = a.ctypes.data, blocks.ctypes.data, c.ctypes.data
    p.m, p.n, p.k = M, n, K
    p.lda, p.ldc = a.strides[0] // a.itemsize, n
    p.ldb_bytes = blocks.strides[0] if ldb_bytes is None else ldb_bytes
    p.trans_b, p.a_f16, p.c_f16 = int(trans_b), int(a.dtype == np.float16), int(c_f16)
    p.w_round_f16, p.acc_f64 = int(w_round_f16), int(acc_f64)
    p.m_begin, p.m_end = (rows if rows is not None else (0, 0))
    lib().orc_gemm_q4_1(C.byref(p))
    return c


def gemm_fp(a, b, *, trans_b=True):
    """Dense fp product of nnops' float routes (f32 x f32 or f16 x f16): the
    exact products of the operands' values summed in float64, rounded once to
    f32 (src/backend/cpu/matmul/matmul_small.cpp, matmul.cpp:57-198 compute
    the same sum in f32; their f16 route also rounds to f16 every 128 k).
    ``b``: [N, K] with trans_b, else [K, N]. Returns f32 [M, N]."""
    a64 = np.asarray(a, dtype=np.float64)
    b64 = np.asarray(b, dtype=np.float64)
    return (a64 @ (b64.T if trans_b else b64)).astype(np.float32)


def fp_linear(a, w, **pass_kw):
    """Linear over a dense weight [n_w, K] of X's type: gemm_fp, then the fp
    output pass (``pass_kw`` as fp_out_pass; gated: the weight's 2n rows)."""
    acc = gemm_fp(a, w, trans_b=True)
    n = w.shape[0] // 2 if pass_kw.get("gated") else w.shape[0]
    return fp_out_pass(acc, n, **pass_kw)


def fp_out_pass(src, n, *, out=None, out_f16=False, bias=None, act=ACT_NONE, act_alpha=0.0, act_beta=1.0,
                min_clip=-np.inf, max_clip=np.inf, add_to=False, residual_pre=False, gated=False,
                gate_act=ACT_SILU, gate_alpha=1.0, gate_beta=0.0, gate_limit=np.inf, matmul_order=False,
                alpha=1.0, beta=0.0):
    """The fp output pass over f32 GEMM results ``src`` [rows, n] (gated:
    [rows, 2n]); ``out`` holds the residual when add_to (f32 or f16, as
    out_f16); ``bias`` in the output's type. ``matmul_order``: MatMul's
    act(clip(alpha src + T(beta old + bias))) (``out`` holds old C).
    Returns the output."""
    src = np.ascontiguousarray(src, dtype=np.float32)
    rows = src.shape[0]
    odt = np.float16 if out_f16 else np.float32
    o = np.zeros((rows, n), dtype=odt) if out is None else np.ascontiguousarray(out, dtype=odt).copy()
    b = None if bias is None else np.ascontiguousarray(bias, dtype=odt)
    p = FpOut()
    p.src, p.ld_src, p.out, p.ld_out = src.ctypes.data, src.shape[1], o.ctypes.data, n
    p.rows, p.n, p.out_f16 = rows, n, int(out_f16)
    p.bias = None if b is None else b.ctypes.data
    p.act, p.act_alpha, p.act_beta, p.min_clip, p.max_clip = act, act_alpha, act_beta, min_clip, max_clip
    p.add_to, p.residual_pre, p.gated, p.gate_act = int(add_to), int(residual_pre), int(gated), gate_act
    p.gate_alpha, p.gate_beta, p.gate_limit = gate_alpha, gate_beta, gate_limit
    p.matmul_order, p.alpha, p.beta = int(matmul_order), alpha, beta
    lib().orc_fp_out_pass(C.byref(p))
    return o


def q4_1_linear(a, blocks, n_w, rows=None, w_round_f16=False, **pass_kw):
    """Linear over a Q4_1 weight [n_w, K] (blocks along K): the f32 dequant
    GEMM (f64 accumulation) and then the fp output pass (``pass_kw`` as
    fp_out_pass; gated: n_w = 2n). ``rows`` = (begin, end): only those rows
    of X (the result has end - begin rows). ``w_round_f16``: the weight decoded
    to f16 first (nnops' packed route for an f16 X past the small-M route)."""
    acc = gemm_q4_1(a, blocks, n_w, trans_b=True, rows=rows, w_round_f16=w_round_f16)
    if rows is not None:
        acc = acc[rows[0]:rows[1]]
        if pass_kw.get("out") is not None:
            pass_kw["out"] = pass_kw["out"][rows[0]:rows[1]]
    n = n_w // 2 if pass_kw.get("gated") else n_w
    return fp_out_pass(acc, n, **pass_kw)


def q4_1_decode(blocks, count):
    out = np.empty(count, dtype=np.float32)
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    lib().orc_q4_1_decode(b.ctypes.data, count, out.ctypes.data)
    return out


def q4_1_quantize(x):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    nb = (x.size + 31) // 32
    out = np.zeros(nb * 20, dtype=np.uint8)
    lib().orc_q4_1_quantize(x.ctypes.data, x.size, out.ctypes.data)
    return out


def qdq_layout(shape, n_params, axis=-1):
    """(inner, dim, segment) of QuantizeLinear / DequantizeLinear for a tensor
    of ``shape`` with ``n_params`` scales: per tensor when n_params <= 1, per
    token for axis < 0, per channel along ``axis`` otherwise
    (src/backend/cpu/quant_linear.cpp:92-118)."""
    numel = int(np.prod(shape)) if len(shape) else 1
    if n_params <= 1:
        return 1, 1, max(numel, 1)
    if axis < 0:
        cols = shape[-1]
        return cols, numel // cols, cols
    inner = int(np.prod(shape[axis + 1:])) if axis + 1 < len(shape) else 1
    return inner, shape[axis], inner


def _params(scale, zero_point):
    s = np.ascontiguousarray(np.atleast_1d(np.asarray(scale, dtype=np.float32)))
    z = None if zero_point is None else np.ascontiguousarray(np.atleast_1d(np.asarray(zero_point)).astype(np.int32))
    return s, z


def quantize_linear(x, scale, zero_point=None, *, out_dtype=np.int8, axis=-1):
    """x: float32/float16 array; scale: f32 scalar or 1-D; zero_point: int
    scalar / 1-D or None. Returns an int8/uint8 array of x's shape."""
    x = np.ascontiguousarray(x)
    assert x.dtype in (np.float32, np.float16)
    s, z = _params(scale, zero_point)
    inner, dim, _ = qdq_layout(x.shape, s.size, axis)
    y = np.zeros(x.shape, dtype=out_dtype)
    lib().orc_quantize_linear(x.ctypes.data, int(x.dtype == np.float16), y.ctypes.data,
                              int(np.dtype(out_dtype) == np.uint8), x.size, s.ctypes.data,
                              _p(z), inner, dim)
    return y


def dequantize_linear(x, scale, zero_point=None, *, out_dtype=np.float32, axis=-1):
    """x: int8/uint8 array. Returns float32/float16 of x's shape."""
    x = np.ascontiguousarray(x)
    assert x.dtype in (np.int8, np.uint8)
    s, z = _params(scale, zero_point)
    inner, dim, seg = qdq_layout(x.shape, s.size, axis)
    y = np.zeros(x.shape, dtype=out_dtype)
    lib().orc_dequantize_linear(x.ctypes.data, int(x.dtype == np.uint8), y.ctypes.data,
                                int(np.dtype(out_dtype) == np.float16), x.size, s.ctypes.data,
                                _p(z), inner, dim, seg)
    return y
