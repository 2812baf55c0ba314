"""Python conveniences over the two C ABIs, for torch tensors on a HIP device.

torch is used only for device memory and streams. Every compute call goes to
libnnops_amd.so; the workspace is allocated here (by torch) only because the
library itself never allocates.
"""
from __future__ import annotations

import ctypes as C
import math

from . import _lib as L

_TORCH_DT = None


def _dt_code(t):
    import torch
    global _TORCH_DT
    if _TORCH_DT is None:
        _TORCH_DT = {torch.float32: L.DT_F32, torch.float16: L.DT_F16, torch.int8: L.DT_S8,
                     torch.uint8: L.DT_U8, torch.int32: L.DT_S32}
    return _TORCH_DT[t.dtype]


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, int):
        return x or None
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    return x.ctypes.data  # host (numpy) table: the caller keeps it alive


def tensor(t, *, dtype=None, shape=None, scale=1.0, zero_point=0, scale_data=None,
           zero_point_data=None, granularity=None, pitch=None):
    """An NnopsTensor over a torch tensor (device memory). The innermost dim
    must be contiguous; the row pitch is taken from stride(-2) unless given.
    ``dtype``/``shape`` override the torch view (q4_1: pass DT_Q4_1 and the
    logical shape in values, the tensor being the uint8 block bytes).
    ``scale_data``/``zero_point_data`` may be host (numpy) or device (torch)."""
    x = L.Tensor()
    shp = list(shape) if shape is not None else list(t.shape)
    x.rank = len(shp)
    for i, d in enumerate(shp):
        x.dims[i] = int(d)
    x.dtype = _dt_code(t) if dtype is None else dtype
    x.data = t.data_ptr() if t is not None else None
    if pitch is not None:
        x.pitch = int(pitch)
    elif t is not None and t.dim() >= 2:
        assert t.stride(-1) == 1, "innermost dim must be contiguous"
        x.pitch = t.stride(-2) * t.element_size()
    x.scale = float(scale)
    x.zero_point = int(zero_point)
    keep = []
    for name, arr in (("scale_data", scale_data), ("zero_point_data", zero_point_data)):
        if arr is None:
            continue
        if hasattr(arr, "data_ptr"):
            setattr(x, name, arr.data_ptr())
        else:
            import numpy as np
            a = np.ascontiguousarray(arr, dtype=np.float32 if name == "scale_data" else np.int32)
            keep.append(a)
            setattr(x, name, a.ctypes.data)
        x.num_scales = len(arr)
    if granularity is not None:
        x.granularity = granularity
    elif scale_data is not None or zero_point_data is not None:
        x.granularity = 1
    x._keep = keep + [t]  # the buffers (device tensor, host tables) must outlive the call
    return x


def _stream_ptr(stream):
    if isinstance(stream, int):
        return stream or None
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def _workspace(nbytes, device):
    import torch
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def _epilogue(ep, act=None, min_clip=-math.inf, max_clip=math.inf, quant=L.EQ_NONE,
              quant_scales=None, quant_zero_points=None, quant_param_count=0, alpha=0.0, beta=1.0):
    ep.type = act or L.EP_NONE
    ep.alpha, ep.beta = alpha, beta
    ep.min_clip, ep.max_clip = min_clip, max_clip
    ep.quant = quant
    ep.quant_scales = _ptr(quant_scales)
    ep.quant_zero_points = _ptr(quant_zero_points)
    ep.quant_param_count = quant_param_count


def _host_tables(scales, zps):
    """Epilogue tables: device tensors pass through; host arrays are made
    contiguous f32/int32 and kept alive by the op (the op stores the pointer)."""
    import numpy as np
    out = []
    for arr, dt in ((scales, np.float32), (zps, np.int32)):
        if arr is None or hasattr(arr, "data_ptr"):
            out.append(arr)
        else:
            out.append(np.ascontiguousarray(arr, dtype=dt))
    return out


class _Op:
    def __init__(self, handle):
        if not handle:
            raise RuntimeError("nnops op creation failed")
        self._h = handle

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            L.lib().nnops_op_destroy(h)
            self._h = None

    @staticmethod
    def _arr(ts):
        ts = list(ts)
        arr = (L.Tensor * max(1, len(ts)))()
        for i, t in enumerate(ts):
            arr[i] = t
        return arr, len(ts)

    def output_desc(self, inputs):
        arr, n = self._arr(inputs)
        out = L.Tensor()
        rc = L.lib().nnops_op_output_desc(self._h, arr, n, C.byref(out))
        if rc != 0:
            raise ValueError(f"output_desc failed: status {rc}")
        return [out.dims[i] for i in range(out.rank)], out.dtype

    def validate(self, inputs, outputs):
        ai, ni = self._arr(inputs)
        ao, no = self._arr(outputs)
        return L.lib().nnops_op_validate(self._h, ai, ni, ao, no)

    def workspace_size(self, inputs, outputs):
        ai, ni = self._arr(inputs)
        ao, no = self._arr(outputs)
        return L.lib().nnops_op_workspace_size(self._h, ai, ni, ao, no)

    def prepack(self, weight, *, stream=None, device="cuda"):
        """prepackWeights: query the packed form of ``weight`` (an NnopsTensor
        from :func:`tensor`), allocate it (torch, device memory) and fill it.
        Returns ``(buffer, packed)`` -- ``packed`` is the NnopsTensor to pass as
        the B / weight input -- or ``(None, None)`` when the weight has no
        packed form."""
        import torch
        ins = (L.Tensor * 1)(weight)
        out = (L.Tensor * 1)()
        rc = L.lib().nnops_op_prepack_weights(self._h, ins, 1, out, 1, None)
        if rc != 0:
            raise ValueError(f"prepack query failed: status {rc}")
        d = out[0]
        if d.rank == 0:
            return None, None
        nbytes = d.dims[0] * d.pitch
        buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
        d.data = buf.data_ptr()
        out[0] = d
        rc = L.lib().nnops_op_prepack_weights(self._h, ins, 1, out, 1, _stream_ptr(stream))
        if rc != 0:
            raise ValueError(f"prepack failed: status {rc}")
        packed = out[0]
        packed._keep = [buf] + list(getattr(weight, "_keep", []))
        return buf, packed

    def compute(self, outputs, inputs, *, stream=None, workspace=None, device="cuda"):
        """Run compute(); allocates a workspace of workspace_size() bytes when
        none is given. Returns the nnops Status code."""
        ai, ni = self._arr(inputs)
        ao, no = self._arr(outputs)
        if workspace is None:
            workspace = _workspace(L.lib().nnops_op_workspace_size(self._h, ai, ni, ao, no), device)
        return L.lib().nnops_op_compute(self._h, ao, no, ai, ni, _stream_ptr(stream), _ptr(workspace))


class MatMul(_Op):
    def __init__(self, *, transpose_a=False, transpose_b=False, output_dtype=L.DT_S32, act=None,
                 min_clip=-math.inf, max_clip=math.inf, quant=L.EQ_NONE, quant_scales=None,
                 quant_zero_points=None, quant_param_count=0, residual_pre_activation=False,
                 requant_round_even=False, float_epilogue=False, act_quant_dtype=L.DT_S8,
                 act_alpha=0.0, act_beta=1.0, alpha=1.0, beta=0.0, backend=L.BACKEND_HIP):
        a = L.MatMulAttrs()
        L.lib().nnops_matmul_attrs_init(C.byref(a))
        a.transpose_a, a.transpose_b = int(transpose_a), int(transpose_b)
        # the product's and old C's scales: read by the fp (q4_1) routes,
        # ignored by the integer ones, as in nnops
        a.alpha, a.beta = alpha, beta
        a.output_dtype = output_dtype
        a.residual_pre_activation = int(residual_pre_activation)
        a.requant_round_even = int(requant_round_even)
        a.float_epilogue = int(float_epilogue)
        a.act_quant_dtype = act_quant_dtype
        self._keep = _host_tables(quant_scales, quant_zero_points)
        _epilogue(a.epilogue, act, min_clip, max_clip, quant, *self._keep, quant_param_count,
                  alpha=act_alpha, beta=act_beta)
        super().__init__(L.lib().nnops_matmul_create(C.byref(a), backend))


class Linear(_Op):
    def __init__(self, *, output_dtype=L.DT_F32, act=None, min_clip=-math.inf, max_clip=math.inf,
                 add_to=False, residual_pre_activation=False, quant=L.EQ_NONE, quant_scales=None,
                 quant_zero_points=None, quant_param_count=0, requant_round_even=False,
                 float_epilogue=False, gated=False, gate_activation=None, gate_alpha=1.0, gate_beta=0.0,
                 gate_limit=math.inf, act_alpha=0.0, act_beta=1.0, backend=L.BACKEND_HIP):
        a = L.LinearAttrs()
        L.lib().nnops_linear_attrs_init(C.byref(a))
        if gate_activation is not None:
            a.gate_activation = gate_activation
        a.gate_alpha, a.gate_beta, a.gate_limit = gate_alpha, gate_beta, gate_limit
        a.output_dtype = output_dtype
        a.add_to = int(add_to)
        a.residual_pre_activation = int(residual_pre_activation)
        a.requant_round_even = int(requant_round_even)
        a.float_epilogue = int(float_epilogue)
        a.gated = int(gated)
        self._keep = _host_tables(quant_scales, quant_zero_points)
        _epilogue(a.epilogue, act, min_clip, max_clip, quant, *self._keep, quant_param_count,
                  alpha=act_alpha, beta=act_beta)
        super().__init__(L.lib().nnops_linear_create(C.byref(a), backend))


class QuantizeLinear(_Op):
    """inputs: x (f32/f16), scale (f32 device tensor), zero point (s8/u8
    device tensor of scale's size); output s8/u8 of x's shape."""

    def __init__(self, *, axis=-1, output_dtype=L.DT_S8, backend=L.BACKEND_HIP):
        a = L.QuantLinearAttrs()
        L.lib().nnops_quant_linear_attrs_init(C.byref(a))
        a.axis, a.output_dtype = axis, output_dtype
        super().__init__(L.lib().nnops_quantize_linear_create(C.byref(a), backend))


class DequantizeLinear(_Op):
    """inputs: x (s8/u8), scale (f32), zero point (s8/u8); output f32/f16."""

    def __init__(self, *, axis=-1, output_dtype=L.DT_F32, backend=L.BACKEND_HIP):
        a = L.QuantLinearAttrs()
        L.lib().nnops_quant_linear_attrs_init(C.byref(a))
        a.axis, a.output_dtype = axis, output_dtype
        super().__init__(L.lib().nnops_dequantize_linear_create(C.byref(a), backend))


def gemm_i8(a, b, c, *, trans_a=False, trans_b=False, bias=None, out_kind=L.OUT_S32,
            s_a=1.0, zp_a=0, s_b=1.0, zp_b=0, s_out=1.0, zp_out=0, s_out_rows=None,
            zp_out_rows=None, act=L.ACT_NONE, round_even=False, float_ep=False,
            min_clip=-math.inf, max_clip=math.inf, add_to=False, residual_pre=False,
            bias_fp=None, act_alpha=0.0, act_beta=1.0,
            m=None, n=None, k=None, workspace=None, stream=None, check=True, noalloc=False):
    """Direct call of nnops_hip_gemm_i8 on torch device tensors. Scales/zero
    points are python scalars or device tensors (per row / per column). An
    f32/f16 destination (OUT_F32 / OUT_F16) takes its bias as `bias_fp`.
    noalloc: call nnops_hip_gemm_i8_noalloc instead (the library's own fixed
    scratch; `workspace` is ignored)."""
    import torch
    g = L.GemmI8Args()
    M = m if m is not None else (a.shape[1] if trans_a else a.shape[0])
    K = k if k is not None else (a.shape[0] if trans_a else a.shape[1])
    N = n if n is not None else (b.shape[0] if trans_b else b.shape[1])
    g.a, g.b, g.c, g.bias = a.data_ptr(), b.data_ptr(), c.data_ptr(), _ptr(bias)
    g.m, g.n, g.k = M, N, K
    g.lda, g.ldb, g.ldc = a.stride(0), b.stride(0), c.stride(0)
    g.trans_a, g.trans_b, g.a_u8 = int(trans_a), int(trans_b), int(a.dtype == torch.uint8)

    def split(v, isf):
        if isinstance(v, torch.Tensor):
            return v.data_ptr(), (1.0 if isf else 0)
        return None, v
    g.s_a, g.s_a_scalar = split(s_a, True)
    g.zp_a, g.zp_a_scalar = split(zp_a, False)
    g.s_b, g.s_b_scalar = split(s_b, True)
    g.zp_b, g.zp_b_scalar = split(zp_b, False)
    g.s_out_rows, g.zp_out_rows = _ptr(s_out_rows), _ptr(zp_out_rows)
    g.s_out, g.zp_out = s_out, zp_out
    g.out_kind, g.act, g.round_even = out_kind, act, int(round_even)
    g.float_ep, g.min_clip, g.max_clip = int(float_ep), min_clip, max_clip
    g.add_to, g.residual_pre = int(add_to), int(residual_pre)
    g.bias_fp, g.act_alpha, g.act_beta = _ptr(bias_fp), act_alpha, act_beta
    lib = L.lib()
    if noalloc:
        rc = lib.nnops_hip_gemm_i8_noalloc(C.byref(g), _stream_ptr(stream))
        if check and rc != 0:
            raise RuntimeError(f"nnops_hip_gemm_i8_noalloc failed: status {rc}")
        return rc
    need = lib.nnops_hip_gemm_i8_workspace_size(C.byref(g))
    if workspace is None:
        workspace = _workspace(need, a.device)
    rc = lib.nnops_hip_gemm_i8(C.byref(g), _ptr(workspace), need, _stream_ptr(stream))
    if check and rc != 0:
        raise RuntimeError(f"nnops_hip_gemm_i8 failed: status {rc}")
    return rc


def gemm_fp(a, b, c, *, trans_b=True, alpha=1.0, workspace=None, stream=None, check=True):
    """Direct call of nnops_hip_gemm_fp: ``a`` f32/f16 [M,K], ``b`` the same
    type [N,K] (trans_b) or [K,N], ``c`` f32/f16 [M,N]: C = alpha A B."""
    import torch
    g = L.GemmFpArgs()
    g.a, g.b, g.c = a.data_ptr(), b.data_ptr(), c.data_ptr()
    g.m, g.k = a.shape
    g.n = b.shape[0] if trans_b else b.shape[1]
    g.lda, g.ldb, g.ldc = a.stride(0), b.stride(0), c.stride(0)
    g.trans_b, g.in_f16 = int(trans_b), int(a.dtype == torch.float16)
    g.out_f16, g.alpha = int(c.dtype == torch.float16), alpha
    lib = L.lib()
    need = lib.nnops_hip_gemm_fp_workspace_size(C.byref(g))
    if workspace is None:
        workspace = _workspace(need, a.device)
    rc = lib.nnops_hip_gemm_fp(C.byref(g), _ptr(workspace), need, _stream_ptr(stream))
    if check and rc != 0:
        raise RuntimeError(f"nnops_hip_gemm_fp failed: status {rc}")
    return rc


def gemm_q4_1(a, b, c, *, n, trans_b=True, ldb_bytes=None, workspace=None, stream=None,
              check=True):
    """Direct call of nnops_hip_gemm_q4_1: ``a`` f16/f32 [M,K], ``b`` uint8 block
    rows (2-D), ``c`` f32/f16 [M,N]."""
    import torch
    g = L.GemmQ41Args()
    g.a, g.b, g.c = a.data_ptr(), b.data_ptr(), c.data_ptr()
    g.m, g.n, g.k = a.shape[0], n, a.shape[1]
    g.lda, g.ldc = a.stride(0), c.stride(0)
    g.ldb_bytes = b.stride(0) if ldb_bytes is None else ldb_bytes
    g.trans_b, g.a_f16 = int(trans_b), int(a.dtype == torch.float16)
    g.out_kind = L.OUT_F16 if c.dtype == torch.float16 else L.OUT_F32
    lib = L.lib()
    need = lib.nnops_hip_gemm_q4_1_workspace_size(C.byref(g))
    if workspace is None:
        workspace = _workspace(need, a.device)
    rc = lib.nnops_hip_gemm_q4_1(C.byref(g), _ptr(workspace), need, _stream_ptr(stream))
    if check and rc != 0:
        raise RuntimeError(f"nnops_hip_gemm_q4_1 failed: status {rc}")
    return rc


def q4_1_quantize(x, out=None, *, stream=None):
    """quantize_q4 on the device: ``x`` a 2-D f32/f16 torch tensor (rows of
    values, any row stride) -> uint8 [rows, ceil(cols/32)*20] llama.cpp
    block_q4_1 rows (``out`` if given). Raises on a rejected call."""
    import torch
    rows, cols = x.shape
    nbb = (cols + 31) // 32 * 20
    if out is None:
        out = torch.empty((rows, nbb), dtype=torch.uint8, device=x.device)
    rc = L.lib().nnops_hip_q4_1_quantize(x.data_ptr(), int(x.dtype == torch.float16), rows, cols, x.stride(0),
                                         out.data_ptr(), out.stride(0), _stream_ptr(stream))
    if rc != 0:
        raise RuntimeError(f"nnops_hip_q4_1_quantize failed: status {rc}")
    return out


def q4_1_dequantize(blocks, cols, out=None, *, dtype=None, stream=None):
    """pack_q4 on the device: uint8 [rows, nb*20] block rows -> f32 (or
    ``dtype`` f16) [rows, cols] (``out`` if given)."""
    import torch
    rows = blocks.shape[0]
    if out is None:
        out = torch.empty((rows, cols), dtype=dtype or torch.float32, device=blocks.device)
    rc = L.lib().nnops_hip_q4_1_dequantize(blocks.data_ptr(), blocks.stride(0), rows, cols, out.data_ptr(),
                                           int(out.dtype == torch.float16), out.stride(0), _stream_ptr(stream))
    if rc != 0:
        raise RuntimeError(f"nnops_hip_q4_1_dequantize failed: status {rc}")
    return out
