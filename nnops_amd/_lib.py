"""ctypes declarations of include/nnops_amd.h and include/nnops_amd_ops.h."""
from __future__ import annotations

import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnnops_amd.so")
DIAG_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnnops_amd_diag.so")

OK, INVALID_ARGUMENT, UNSUPPORTED, NOT_INITIALIZED, OUT_OF_MEMORY, INTERNAL = range(6)
OUT_S32, OUT_S8, OUT_U8, OUT_F32, OUT_F16 = range(5)
(ACT_NONE, ACT_RELU, ACT_GELU, ACT_SIGMOID, ACT_TANH, ACT_LEAKY_RELU, ACT_SILU, ACT_HARDSWISH, ACT_ELU,
 ACT_RELU6) = range(10)
DT_F32, DT_F16, DT_BF16, DT_S8, DT_U8, DT_S32 = 0, 1, 2, 3, 4, 5
DT_Q4_1 = 11
LAYOUT_DENSE, LAYOUT_PACKED_B_HIP = 12, 18
BACKEND_CPU, BACKEND_CUDA, BACKEND_HIP = 0, 1, 4
# EpilogueActivateType / EpilogueQuantType values
EP_NONE, EP_RELU, EP_GELU, EP_SIGMOID, EP_TANH = 0, 1, 2, 3, 4
EP_LEAKY_RELU, EP_SILU, EP_HARDSWISH, EP_ELU, EP_RELU6 = 5, 6, 7, 8, 9
EQ_NONE, EQ_REQUANTIZE, EQ_DEQUANTIZE = 0, 1, 2


class GemmI8Args(C.Structure):
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
        ("bias_fp", C.c_void_p), ("act_alpha", C.c_float), ("act_beta", C.c_float),
        ("b_col_sums", C.c_void_p),
    ]


class QdqArgs(C.Structure):
    _fields_ = [
        ("x", C.c_void_p), ("y", C.c_void_p),
        ("rows", C.c_int64), ("cols", C.c_int64), ("ld_x", C.c_int64), ("ld_y", C.c_int64),
        ("x_kind", C.c_int32), ("y_kind", C.c_int32), ("zp_kind", C.c_int32),
        ("scale", C.c_void_p), ("zero_point", C.c_void_p), ("scale_scalar", C.c_float),
        ("zp_scalar", C.c_int32), ("inner", C.c_int64), ("dim", C.c_int64), ("segment", C.c_int64),
    ]


class GemmQ41Args(C.Structure):
    _fields_ = [
        ("a", C.c_void_p), ("b", C.c_void_p), ("c", C.c_void_p),
        ("m", C.c_int64), ("n", C.c_int64), ("k", C.c_int64),
        ("lda", C.c_int64), ("ldc", C.c_int64), ("ldb_bytes", C.c_int64),
        ("trans_b", C.c_int32), ("a_f16", C.c_int32), ("out_kind", C.c_int32),
        ("b_soa", C.c_int32), ("b_dm", C.c_void_p), ("ldb_dm", C.c_int64),
    ]


class GemmFpArgs(C.Structure):
    _fields_ = [
        ("a", C.c_void_p), ("b", C.c_void_p), ("c", C.c_void_p),
        ("m", C.c_int64), ("n", C.c_int64), ("k", C.c_int64),
        ("lda", C.c_int64), ("ldb", C.c_int64), ("ldc", C.c_int64),
        ("trans_b", C.c_int32), ("in_f16", C.c_int32), ("out_f16", C.c_int32), ("alpha", C.c_float),
    ]


class Tensor(C.Structure):
    _fields_ = [
        ("rank", C.c_int64), ("dims", C.c_int64 * 8), ("dtype", C.c_int32),
        ("data", C.c_void_p), ("pitch", C.c_int64),
        ("granularity", C.c_int32), ("scale", C.c_float), ("zero_point", C.c_int32),
        ("scale_data", C.c_void_p), ("zero_point_data", C.c_void_p), ("num_scales", C.c_int64),
        ("layout", C.c_int32),
    ]


class Epilogue(C.Structure):
    _fields_ = [
        ("type", C.c_int32), ("alpha", C.c_float), ("beta", C.c_float),
        ("min_clip", C.c_float), ("max_clip", C.c_float),
        ("quant", C.c_int32), ("quant_scales", C.c_void_p), ("quant_zero_points", C.c_void_p),
        ("quant_param_count", C.c_int64),
    ]


class MatMulAttrs(C.Structure):
    _fields_ = [
        ("transpose_a", C.c_int32), ("transpose_b", C.c_int32),
        ("alpha", C.c_float), ("beta", C.c_float),
        ("residual_pre_activation", C.c_int32), ("output_dtype", C.c_int32),
        ("epilogue", Epilogue),
        ("requant_round_even", C.c_int32), ("float_epilogue", C.c_int32),
        ("act_quant_dtype", C.c_int32),
    ]


class QuantLinearAttrs(C.Structure):
    _fields_ = [("axis", C.c_int64), ("output_dtype", C.c_int32)]


class LinearAttrs(C.Structure):
    _fields_ = [
        ("epilogue", Epilogue),
        ("add_to", C.c_int32), ("residual_pre_activation", C.c_int32),
        ("output_dtype", C.c_int32), ("gated", C.c_int32),
        ("requant_round_even", C.c_int32), ("float_epilogue", C.c_int32),
        ("gate_activation", C.c_int32), ("gate_alpha", C.c_float), ("gate_beta", C.c_float),
        ("gate_limit", C.c_float),
        ("matmul_order", C.c_int32), ("alpha", C.c_float), ("beta", C.c_float),
    ]


class FpOutArgs(C.Structure):
    _fields_ = [
        ("src", C.c_void_p), ("ld_src", C.c_int64), ("out", C.c_void_p), ("ld_out", C.c_int64),
        ("rows", C.c_int64), ("n", C.c_int64), ("out_f16", C.c_int32), ("bias", C.c_void_p),
        ("act", C.c_int32), ("act_alpha", C.c_float), ("act_beta", C.c_float),
        ("min_clip", C.c_float), ("max_clip", C.c_float),
        ("add_to", C.c_int32), ("residual_pre", C.c_int32), ("gated", C.c_int32),
        ("gate_act", C.c_int32), ("gate_alpha", C.c_float), ("gate_beta", C.c_float), ("gate_limit", C.c_float),
        ("matmul_order", C.c_int32), ("alpha", C.c_float), ("beta", C.c_float),
    ]


# Every symbol the two headers declare, with its ctypes signature.
SIGNATURES = {
    "nnops_hip_gemm_i8_workspace_size": (C.c_size_t, [C.POINTER(GemmI8Args)]),
    "nnops_hip_gemm_i8": (C.c_int, [C.POINTER(GemmI8Args), C.c_void_p, C.c_size_t, C.c_void_p]),
    "nnops_hip_gemm_i8_noalloc": (C.c_int, [C.POINTER(GemmI8Args), C.c_void_p]),
    "nnops_hip_gemm_q4_1_workspace_size": (C.c_size_t, [C.POINTER(GemmQ41Args)]),
    "nnops_hip_gemm_q4_1": (C.c_int, [C.POINTER(GemmQ41Args), C.c_void_p, C.c_size_t, C.c_void_p]),
    "nnops_hip_gemm_fp_workspace_size": (C.c_size_t, [C.POINTER(GemmFpArgs)]),
    "nnops_hip_gemm_fp": (C.c_int, [C.POINTER(GemmFpArgs), C.c_void_p, C.c_size_t, C.c_void_p]),
    "nnops_hip_fp_output_pass": (C.c_int, [C.POINTER(FpOutArgs), C.c_void_p]),
    "nnops_hip_gemm_q4_1_fused": (C.c_int, [C.POINTER(GemmQ41Args), C.POINTER(FpOutArgs), C.c_void_p]),
    "nnops_hip_build_info": (C.c_char_p, []),
    "nnops_hip_time_next_launch": (C.c_int, [C.c_void_p, C.c_void_p]),
    "nnops_hip_prepack_i8_bytes": (C.c_size_t, [C.c_int64, C.c_int64]),
    "nnops_hip_prepack_q4_1_bytes": (C.c_size_t, [C.c_int64, C.c_int64]),
    "nnops_hip_prepack_q4_1": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int32, C.c_void_p,
                                         C.c_void_p]),
    "nnops_hip_prepack_i8": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int32, C.c_void_p,
                                       C.c_void_p]),
    "nnops_hip_q4_1_quantize": (C.c_int, [C.c_void_p, C.c_int32, C.c_int64, C.c_int64, C.c_int64, C.c_void_p,
                                          C.c_int64, C.c_void_p]),
    "nnops_hip_q4_1_dequantize": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_int32,
                                            C.c_int64, C.c_void_p]),
    "nnops_hip_quantize_linear": (C.c_int, [C.POINTER(QdqArgs), C.c_void_p]),
    "nnops_hip_dequantize_linear": (C.c_int, [C.POINTER(QdqArgs), C.c_void_p]),
    "nnops_matmul_attrs_init": (None, [C.POINTER(MatMulAttrs)]),
    "nnops_linear_attrs_init": (None, [C.POINTER(LinearAttrs)]),
    "nnops_matmul_create": (C.c_void_p, [C.POINTER(MatMulAttrs), C.c_int32]),
    "nnops_linear_create": (C.c_void_p, [C.POINTER(LinearAttrs), C.c_int32]),
    "nnops_quant_linear_attrs_init": (None, [C.POINTER(QuantLinearAttrs)]),
    "nnops_quantize_linear_create": (C.c_void_p, [C.POINTER(QuantLinearAttrs), C.c_int32]),
    "nnops_dequantize_linear_create": (C.c_void_p, [C.POINTER(QuantLinearAttrs), C.c_int32]),
    "nnops_op_destroy": (None, [C.c_void_p]),
    "nnops_op_prepack_weights": (C.c_int, [C.c_void_p, C.POINTER(Tensor), C.c_int32, C.POINTER(Tensor), C.c_int32,
                                           C.c_void_p]),
    "nnops_op_output_desc": (C.c_int, [C.c_void_p, C.POINTER(Tensor), C.c_int32, C.POINTER(Tensor)]),
    "nnops_op_validate": (C.c_int, [C.c_void_p, C.POINTER(Tensor), C.c_int32, C.POINTER(Tensor), C.c_int32]),
    "nnops_op_workspace_size": (C.c_size_t, [C.c_void_p, C.POINTER(Tensor), C.c_int32,
                                             C.POINTER(Tensor), C.c_int32]),
    "nnops_op_compute": (C.c_int, [C.c_void_p, C.POINTER(Tensor), C.c_int32, C.POINTER(Tensor),
                                   C.c_int32, C.c_void_p, C.c_void_p]),
}

_lib = None


def load(path: str = LIB_PATH):
    """Load the library (raises if it was not built: there is no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise RuntimeError(
                f"nnops_amd native library missing: {path}; build it with `python -m nnops_amd.build`")
        # One HIP runtime per process: torch ships its own libamdhip64 (same
        # soname as ROCm's). Loaded after torch, this library binds to that
        # copy; loaded first, it would bring in ROCm's and torch would then add
        # its own beside it, so device pointers from one runtime would be
        # unknown to the other. Import torch first when it is installed.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        lib_ = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib_, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib_
    return _lib


def lib():
    return load()


# include/nnops_amd_diag.h: measurement probes in their own library (bench only)
DIAG_SIGNATURES = {
    "nnops_hip_diag_mfma_i8": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "nnops_hip_diag_stream_read": (C.c_int, [C.c_void_p, C.c_int64, C.c_void_p, C.c_int, C.c_void_p]),
    "nnops_hip_diag_empty": (C.c_int, [C.c_void_p, C.c_void_p]),
}
_diag = None


def diag_lib():
    """The probe library (libnnops_amd_diag.so), loaded after the product one."""
    global _diag
    if _diag is None:
        load()
        if not os.path.exists(DIAG_PATH):
            raise RuntimeError(f"probe library missing: {DIAG_PATH}; build it with `python -m nnops_amd.build`")
        d = C.CDLL(DIAG_PATH)
        for name, (res, args) in DIAG_SIGNATURES.items():
            fn = getattr(d, name)
            fn.restype = res
            fn.argtypes = args
        _diag = d
    return _diag
