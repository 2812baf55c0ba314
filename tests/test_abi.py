"""The C ABI library without a GPU: it loads, exports every symbol the public
headers declare, and the descriptor-only half of the operator contract
(output descriptors, validate, workspace sizes, rejected calls) behaves like
nnops'. No call here reaches a kernel launch."""
from __future__ import annotations

import ctypes as C
import os
import re

import pytest

import nnops_amd as na
from nnops_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in ("nnops_amd.h", "nnops_amd_ops.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(nnops_\w+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    lib = na.lib()
    names = declared_symbols()
    assert len(names) >= 14
    for n in sorted(names):
        assert hasattr(lib, n), n
        assert n in L.SIGNATURES, f"{n} has no ctypes signature"


def test_probe_library_is_separate():
    """The measurement probes live in libnnops_amd_diag.so, declared by
    nnops_amd_diag.h; the product library exports none of them."""
    text = open(os.path.join(ROOT, "include", "nnops_amd_diag.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = {m.group(1) for m in re.finditer(r"\b(nnops_\w+)\s*\(", text)}
    assert names == set(L.DIAG_SIGNATURES)
    d = L.diag_lib()
    for n in names:
        assert hasattr(d, n), n
        assert not hasattr(na.lib(), n), n


def test_build_info():
    assert b"gfx950" in na.lib().nnops_hip_build_info()


def test_time_next_launch_arguments():
    """The timing hook takes both events or neither; it launches nothing."""
    lib = na.lib()
    assert lib.nnops_hip_time_next_launch(C.c_void_p(16), None) == na.INVALID_ARGUMENT
    assert lib.nnops_hip_time_next_launch(None, C.c_void_p(16)) == na.INVALID_ARGUMENT
    assert lib.nnops_hip_time_next_launch(None, None) == na.OK


def test_gemm_i8_rejects_before_any_launch():
    lib = na.lib()
    g = na.GemmI8Args()
    assert lib.nnops_hip_gemm_i8(None, None, 0, None) == na.INVALID_ARGUMENT
    g.m, g.n, g.k = 4, 4, 4
    assert lib.nnops_hip_gemm_i8(C.byref(g), None, 0, None) == na.INVALID_ARGUMENT  # null data
    g.a = g.b = g.c = 16  # never dereferenced: every rejection below happens first
    g.lda, g.ldb, g.ldc = 4, 4, 4
    g.out_kind = 7                       # no such destination
    assert lib.nnops_hip_gemm_i8(C.byref(g), None, 0, None) == na.UNSUPPORTED
    g.out_kind = na.OUT_S8
    g.act = na.ACT_SIGMOID               # the requantizing pass honours Relu (and Gelu via float_ep) only
    assert lib.nnops_hip_gemm_i8(C.byref(g), None, 0, None) == na.UNSUPPORTED
    g.act = na.ACT_NONE
    g.out_kind = na.OUT_F32
    g.bias = 16                          # an f32 destination takes its bias as bias_fp
    assert lib.nnops_hip_gemm_i8(C.byref(g), None, 0, None) == na.INVALID_ARGUMENT
    g.bias = None
    g.out_kind = na.OUT_S32
    g.float_ep = 1
    assert lib.nnops_hip_gemm_i8(C.byref(g), None, 0, None) == na.UNSUPPORTED
    g.float_ep = 0
    g.lda = 3
    assert lib.nnops_hip_gemm_i8(C.byref(g), None, 0, None) == na.INVALID_ARGUMENT
    g.lda = 4
    g.k = 70000
    g.lda = g.ldb = 70000
    assert lib.nnops_hip_gemm_i8(C.byref(g), None, 0, None) == na.UNSUPPORTED
    # a [K,N] B needs a staging workspace: missing -> not_initialized
    g.k, g.lda, g.ldb = 4, 4, 4
    g.trans_b = 0
    assert lib.nnops_hip_gemm_i8_workspace_size(C.byref(g)) > 0
    assert lib.nnops_hip_gemm_i8(C.byref(g), None, 0, None) == na.NOT_INITIALIZED
    # empty problem: ok, nothing to do
    g.m = 0
    assert lib.nnops_hip_gemm_i8(C.byref(g), None, 0, None) == na.OK


def test_gemm_q4_1_rejects_before_any_launch():
    lib = na.lib()
    g = na.GemmQ41Args()
    g.m, g.n, g.k = 2, 64, 64
    g.a = g.b = g.c = 16
    g.lda, g.ldc = 64, 64
    g.trans_b = 1
    g.ldb_bytes = 40
    g.out_kind = na.OUT_S8
    assert lib.nnops_hip_gemm_q4_1(C.byref(g), None, 0, None) == na.UNSUPPORTED
    g.out_kind = na.OUT_F32
    g.ldb_bytes = 39  # shorter than one row of blocks
    assert lib.nnops_hip_gemm_q4_1(C.byref(g), None, 0, None) == na.INVALID_ARGUMENT
    g.ldb_bytes = 42  # not a multiple of 4
    assert lib.nnops_hip_gemm_q4_1(C.byref(g), None, 0, None) == na.INVALID_ARGUMENT
    # the prepacked planes (b_soa) have fixed block-column pitches, ceil(K/8)
    # * 128 nibble bytes and K rounded up to 64 d|m dwords: every kernel
    # places the block columns by them, so a padded pitch is rejected rather
    # than read two different ways (K = 64: 1024 bytes, 64 dwords)
    g.trans_b, g.b_soa, g.b_dm = 0, 1, 4096
    g.ldb_bytes, g.ldb_dm = 1024 + 128, 64
    g.m = 0  # an empty problem returns before the argument checks: ok
    assert lib.nnops_hip_gemm_q4_1(C.byref(g), None, 0, None) == na.OK
    g.m = 2
    assert lib.nnops_hip_gemm_q4_1(C.byref(g), None, 0, None) == na.INVALID_ARGUMENT
    g.ldb_bytes, g.ldb_dm = 1024, 128
    assert lib.nnops_hip_gemm_q4_1(C.byref(g), None, 0, None) == na.INVALID_ARGUMENT
    g.ldb_bytes, g.ldb_dm = 32, 64   # the old nbn * 16 row pitch
    assert lib.nnops_hip_gemm_q4_1(C.byref(g), None, 0, None) == na.INVALID_ARGUMENT


def test_gemm_q4_1_fused_declines_before_any_launch():
    """nnops_hip_gemm_q4_1_fused takes only the blocks-along-K ring route and
    answers NNOPS_UNSUPPORTED, launching nothing, for the others (the caller
    then runs the two-step form); missing arguments are invalid."""
    from nnops_amd._lib import FpOutArgs
    lib = na.lib()
    g = na.GemmQ41Args()
    fo = FpOutArgs()
    assert lib.nnops_hip_gemm_q4_1_fused(None, C.byref(fo), None) == na.INVALID_ARGUMENT
    assert lib.nnops_hip_gemm_q4_1_fused(C.byref(g), None, None) == na.INVALID_ARGUMENT
    g.m, g.n, g.k = 256, 512, 256
    g.a = g.b = 256
    g.lda, g.ldb_bytes, g.a_f16, g.trans_b = 256, 160, 1, 1
    fo.out, fo.ld_out, fo.rows, fo.n = 256, 512, 256, 512
    for field, value in (("trans_b", 0), ("a_f16", 0), ("m", 2), ("m", 16), ("k", 96), ("lda", 260)):
        old = getattr(g, field)
        setattr(g, field, value)
        assert lib.nnops_hip_gemm_q4_1_fused(C.byref(g), C.byref(fo), None) == na.UNSUPPORTED, field
        setattr(g, field, old)
    # the pass's own checks: an unknown gate activation, a row count other than M
    fo.gated, fo.gate_act, fo.n = 1, na.ACT_HARDSWISH, 256
    assert lib.nnops_hip_gemm_q4_1_fused(C.byref(g), C.byref(fo), None) == na.UNSUPPORTED
    fo.gate_act, fo.rows = na.ACT_SILU, 255
    assert lib.nnops_hip_gemm_q4_1_fused(C.byref(g), C.byref(fo), None) == na.INVALID_ARGUMENT


def test_gemm_fp_rejects_before_any_launch():
    lib = na.lib()
    g = na.GemmFpArgs()
    g.m, g.n, g.k = 64, 64, 64
    g.a = g.b = g.c = 16
    g.lda, g.ldb, g.ldc = 64, 64, 64
    g.trans_b, g.in_f16, g.alpha = 1, 1, 1.0
    g.lda = 63                                   # shorter than K
    assert lib.nnops_hip_gemm_fp(C.byref(g), None, 0, None) == na.INVALID_ARGUMENT
    g.lda, g.ldc = 64, 32                        # C rows shorter than N
    assert lib.nnops_hip_gemm_fp(C.byref(g), None, 0, None) == na.INVALID_ARGUMENT
    g.ldc, g.trans_b, g.ldb, g.n = 64, 0, 64, 96  # [K,N] B rows shorter than N
    assert lib.nnops_hip_gemm_fp(C.byref(g), None, 0, None) == na.INVALID_ARGUMENT
    g.c = None
    assert lib.nnops_hip_gemm_fp(C.byref(g), None, 0, None) == na.INVALID_ARGUMENT
    g.m = 0                                      # an empty problem: ok
    assert lib.nnops_hip_gemm_fp(C.byref(g), None, 0, None) == na.OK
    # a split [K,N] GEMV needs its partials: no workspace is not_initialized
    g.m, g.n, g.ldb, g.ldc, g.k, g.lda, g.c = 1, 4096, 4096, 4096, 4096, 4096, 16
    assert lib.nnops_hip_gemm_fp_workspace_size(C.byref(g)) > 0
    assert lib.nnops_hip_gemm_fp(C.byref(g), None, 0, None) == na.NOT_INITIALIZED


def desc(shape, dtype):
    t = na.Tensor()
    t.rank = len(shape)
    for i, d in enumerate(shape):
        t.dims[i] = d
    t.dtype = dtype
    t.scale = 1.0
    return t


def test_matmul_output_desc_rules():
    # int8 pair -> output_dtype (src/ops/matmul.cpp:49-58)
    op = na.MatMul(output_dtype=na.DT_S8)
    shape, dt = op.output_desc([desc([2, 3], na.DT_S8), desc([3, 5], na.DT_S8)])
    assert shape == [2, 5] and dt == na.DT_S8
    op = na.MatMul(transpose_b=True)
    shape, dt = op.output_desc([desc([7, 9], na.DT_U8), desc([4, 9], na.DT_S8)])
    assert shape == [7, 4] and dt == na.DT_S32
    # batch broadcast
    shape, _ = op.output_desc([desc([3, 1, 7, 9], na.DT_S8), desc([5, 4, 9], na.DT_S8)])
    assert shape == [3, 5, 7, 4]
    # fp x q4_1 follows A
    op = na.MatMul(transpose_b=True)
    shape, dt = op.output_desc([desc([1, 64], na.DT_F16), desc([10, 64], na.DT_Q4_1)])
    assert shape == [1, 10] and dt == na.DT_F16


def test_linear_output_desc_rules():
    # int8: output_dtype when known, default f32 (src/ops/linear.cpp:29-47)
    op = na.Linear()
    shape, dt = op.output_desc([desc([2, 5, 8], na.DT_S8), desc([6, 8], na.DT_S8)])
    assert shape == [2, 5, 6] and dt == na.DT_F32
    op = na.Linear(output_dtype=na.DT_S8)
    _, dt = op.output_desc([desc([4, 8], na.DT_S8), desc([6, 8], na.DT_S8)])
    assert dt == na.DT_S8


def test_validate_and_workspace():
    op = na.MatMul(output_dtype=na.DT_S8)
    ins = [desc([4, 8], na.DT_S8), desc([8, 6], na.DT_S8)]
    outs = [desc([4, 6], na.DT_S8)]
    assert op.validate(ins, outs) == na.OK
    assert op.validate([desc([4, 8], na.DT_S8), desc([7, 6], na.DT_S8)], outs) == na.INVALID_ARGUMENT
    assert op.validate(ins[:1], outs) == na.INVALID_ARGUMENT
    assert op.validate([desc([8], na.DT_S8), ins[1]], outs) == na.INVALID_ARGUMENT
    # honest, non-zero: staging for the QuantParams tables + B transpose
    ws = op.workspace_size(ins, outs)
    assert ws >= 8 * 6
    op_t = na.MatMul(output_dtype=na.DT_S8, transpose_b=True)
    ws_t = op_t.workspace_size([desc([4, 8], na.DT_S8), desc([6, 8], na.DT_S8)], outs)
    assert 0 < ws_t < ws


def test_compute_rejections_without_gpu():
    ins = [desc([4, 8], na.DT_S8), desc([8, 6], na.DT_S8)]
    ins[0].data = ins[1].data = 256
    out = desc([4, 6], na.DT_S8)
    out.data = 512
    # backend with no kernels -> unsupported (dispatch.hpp:93-96 in nnops)
    assert na.MatMul(output_dtype=na.DT_S8, backend=na.BACKEND_CPU).compute([out], ins, stream=0, workspace=0) == na.UNSUPPORTED
    # wrong counts / empty view / K mismatch -> invalid_argument
    op = na.MatMul(output_dtype=na.DT_S8)
    assert op.compute([out], ins[:1], stream=0, workspace=0) == na.INVALID_ARGUMENT
    bad = desc([9, 6], na.DT_S8)
    bad.data = 256
    assert op.compute([out], [ins[0], bad], stream=0, workspace=0) == na.INVALID_ARGUMENT
    empty = desc([4, 8], na.DT_S8)
    assert op.compute([out], [empty, ins[1]], stream=0, workspace=0) == na.INVALID_ARGUMENT
    # output dtype disagreeing with output_dtype
    o32 = desc([4, 6], na.DT_S32)
    o32.data = 512
    assert op.compute([o32], ins, stream=0, workspace=0) == na.INVALID_ARGUMENT
    # gated Linear has no quantized route
    assert na.Linear(gated=True).validate([desc([4, 8], na.DT_S8), desc([6, 8], na.DT_S8)],
                                          [desc([4, 6], na.DT_F32)]) == na.UNSUPPORTED


def test_fp_activation_matmul_descriptors():
    # fp A x s8 B follows A's dtype; workspace holds A_q plus the int8 call's
    op = na.MatMul(act_quant_dtype=na.DT_U8)
    ins = [desc([2, 4, 64], na.DT_F16), desc([64, 32], na.DT_S8)]
    shape, dt = op.output_desc(ins)
    assert shape == [2, 4, 32] and dt == na.DT_F16
    assert op.workspace_size(ins, [desc([2, 4, 32], na.DT_F16)]) >= 2 * 4 * 64
    # dequantizing destinations of the int8 pair
    shape, dt = na.MatMul(output_dtype=na.DT_F16).output_desc([desc([3, 8], na.DT_S8), desc([8, 5], na.DT_S8)])
    assert shape == [3, 5] and dt == na.DT_F16


def test_quant_linear_descriptors_and_validate():
    # quant_linear.hpp: same shape, output_dtype; dequantize resolves non-float to f32
    q = na.QuantizeLinear(output_dtype=na.DT_U8)
    ins = [desc([3, 5, 7], na.DT_F32), desc([15], na.DT_F32), desc([15], na.DT_U8)]
    shape, dt = q.output_desc(ins)
    assert shape == [3, 5, 7] and dt == na.DT_U8
    assert q.validate(ins, [desc([3, 5, 7], na.DT_U8)]) == na.OK
    assert q.validate(ins, [desc([3, 5, 7], na.DT_S32)]) == na.INVALID_ARGUMENT
    assert q.validate([desc([3, 5, 7], na.DT_S32)] + ins[1:], [desc([3, 5, 7], na.DT_U8)]) == na.UNSUPPORTED
    assert q.validate([ins[0], desc([15], na.DT_F16), ins[2]], [desc([3, 5, 7], na.DT_U8)]) == na.INVALID_ARGUMENT
    assert q.validate(ins[:2], [desc([3, 5, 7], na.DT_U8)]) == na.INVALID_ARGUMENT
    d = na.DequantizeLinear(output_dtype=na.DT_S8)
    _, dt = d.output_desc([desc([4, 4], na.DT_S8), desc([1], na.DT_F32), desc([1], na.DT_S8)])
    assert dt == na.DT_F32
    d16 = na.DequantizeLinear(output_dtype=na.DT_F16)
    assert d16.validate([desc([4, 4], na.DT_S8), desc([1], na.DT_F32), desc([1], na.DT_S8)],
                        [desc([4, 4], na.DT_F16)]) == na.OK
    # backend with no kernels
    x = desc([4], na.DT_F32)
    x.data = 256
    s = desc([1], na.DT_F32)
    s.data = 256
    z = desc([1], na.DT_S8)
    z.data = 256
    o = desc([4], na.DT_S8)
    o.data = 512
    assert na.QuantizeLinear(backend=na.BACKEND_CPU).compute([o], [x, s, z], stream=0, workspace=0) \
        == na.UNSUPPORTED


def test_prepack_query_descriptor():
    # query: [N, K] s8 PackedBHip pitched at ceil(bytes / N) (no launch); non-s8 answers empty
    lib = na.lib()
    op = na.MatMul(output_dtype=na.DT_S8)             # B [K, N]
    w = desc([300, 100], na.DT_S8)
    ins = (L.Tensor * 1)(w)
    out = (L.Tensor * 1)()
    assert lib.nnops_op_prepack_weights(op._h, ins, 1, out, 1, None) == na.OK
    kp = 384
    nbytes = ((100 * kp + 255) // 256) * 256 + 4 * 100
    assert out[0].rank == 2 and out[0].dims[0] == 100 and out[0].dims[1] == 300
    assert out[0].dtype == na.DT_S8 and out[0].layout == L.LAYOUT_PACKED_B_HIP
    assert out[0].pitch == -(-nbytes // 100)
    s8packed = out[0]
    # K must be A's exactly: a smaller K in the same 128-padded row is rejected too
    assert op.validate([desc([7, 300], na.DT_S8), s8packed], [desc([7, 100], na.DT_S32)]) == na.OK
    assert op.validate([desc([7, 290], na.DT_S8), s8packed], [desc([7, 100], na.DT_S32)]) \
        == na.INVALID_ARGUMENT
    assert lib.nnops_hip_prepack_i8_bytes(300, 100) == nbytes
    # Linear: the weight is [N, K]
    lop = na.Linear(output_dtype=na.DT_S8)
    ins = (L.Tensor * 1)(desc([100, 300], na.DT_S8))
    out = (L.Tensor * 1)()
    assert lib.nnops_op_prepack_weights(lop._h, ins, 1, out, 1, None) == na.OK
    assert out[0].dims[0] == 100 and out[0].dims[1] == 300 and out[0].pitch == -(-nbytes // 100)
    # q4_1 / f32 weights: no packed form
    ins = (L.Tensor * 1)(desc([64, 16], na.DT_F32))
    out = (L.Tensor * 1)()
    assert lib.nnops_op_prepack_weights(op._h, ins, 1, out, 1, None) == na.OK
    assert out[0].rank == 0
    # q4_1 with blocks along N ([K, N], transpose_b false): PackedBHip q4_1
    # [N, K], pitched at whole blocks so that N rows cover the two planes
    q_bytes = lib.nnops_hip_prepack_q4_1_bytes(256, 100)
    nbn = 4
    assert q_bytes == ((nbn * 32 * 128 + 255) // 256) * 256 + nbn * 256 * 4
    qop = na.MatMul(transpose_b=False)
    ins = (L.Tensor * 1)(desc([256, 100], na.DT_Q4_1))
    out = (L.Tensor * 1)()
    assert lib.nnops_op_prepack_weights(qop._h, ins, 1, out, 1, None) == na.OK
    assert out[0].rank == 2 and out[0].dims[0] == 100 and out[0].dims[1] == 256
    assert out[0].dtype == na.DT_Q4_1 and out[0].layout == L.LAYOUT_PACKED_B_HIP
    assert out[0].pitch == 20 * max(256 // 32, -(-q_bytes // (100 * 20)))
    qpacked = out[0]
    shape, dt = qop.output_desc([desc([7, 256], na.DT_F16), qpacked])
    assert shape == [7, 100] and dt == na.DT_F16
    # A with a larger or a smaller K than the blob was packed for (the d|m
    # plane's offset depends on K)
    assert qop.validate([desc([7, 4096], na.DT_F16), qpacked], [desc([7, 100], na.DT_F16)]) \
        == na.INVALID_ARGUMENT
    assert qop.validate([desc([7, 248], na.DT_F16), qpacked], [desc([7, 100], na.DT_F16)]) \
        == na.INVALID_ARGUMENT
    # blocks along K (transpose_b, and Linear's [N, K] weight): no packed form
    tb = na.MatMul(transpose_b=True)
    ins = (L.Tensor * 1)(desc([100, 256], na.DT_Q4_1))
    out = (L.Tensor * 1)()
    assert lib.nnops_op_prepack_weights(tb._h, ins, 1, out, 1, None) == na.OK
    assert out[0].rank == 0
    lq = na.Linear()
    out = (L.Tensor * 1)()
    assert lib.nnops_op_prepack_weights(lq._h, ins, 1, out, 1, None) == na.OK
    assert out[0].rank == 0
    assert lib.nnops_hip_prepack_q4_1(None, 256, 100, 80, 1, None, None) == na.UNSUPPORTED
    # a packed B: output descriptor from its N and A's K; a K other than the
    # packed one, or a pitch too small for the blob, is rejected
    packed = desc([100, 300], na.DT_S8)
    packed.layout = L.LAYOUT_PACKED_B_HIP
    packed.pitch = -(-nbytes // 100)
    shape, dt = op.output_desc([desc([7, 300], na.DT_S8), packed])
    assert shape == [7, 100] and dt == na.DT_S8
    assert op.validate([desc([7, 300], na.DT_S8), packed], [desc([7, 100], na.DT_S8)]) == na.OK
    assert op.validate([desc([7, 600], na.DT_S8), packed], [desc([7, 100], na.DT_S8)]) == na.INVALID_ARGUMENT
    packed.pitch = 300
    assert op.validate([desc([7, 300], na.DT_S8), packed], [desc([7, 100], na.DT_S8)]) == na.INVALID_ARGUMENT


def test_q4_1_codec_rejects_before_any_launch():
    lib = na.lib()
    assert lib.nnops_hip_q4_1_quantize(16, 0, 2, 64, 32, 16, 40, None) == na.INVALID_ARGUMENT   # ld_src < cols
    assert lib.nnops_hip_q4_1_quantize(16, 0, 2, 64, 64, 16, 38, None) == na.INVALID_ARGUMENT   # pitch < 40
    assert lib.nnops_hip_q4_1_quantize(None, 0, 2, 64, 64, 16, 40, None) == na.INVALID_ARGUMENT
    assert lib.nnops_hip_q4_1_quantize(None, 0, 0, 64, 64, None, 40, None) == na.OK              # empty
    assert lib.nnops_hip_q4_1_dequantize(16, 36, 2, 64, 16, 0, 64, None) == na.INVALID_ARGUMENT
