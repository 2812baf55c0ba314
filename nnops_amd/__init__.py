"""nnops_amd — MI355X (gfx950) quantized-matmul path with nnops' operator API.

The product is ``libnnops_amd.so`` (built in-tree by ``nnops_amd.build``): HIP
kernels behind two C ABIs, ``include/nnops_amd.h`` (kernel launch boundary)
and ``include/nnops_amd_ops.h`` (the MatMul / Linear / QuantizeLinear / DequantizeLinear operator
contract). This
package only binds them with ctypes for Python callers and tests; there is no
Python or CPU fallback: a missing library raises.
"""
from ._lib import (  # noqa: F401
    lib, load, LIB_PATH,
    GemmI8Args, GemmQ41Args, GemmFpArgs, QdqArgs, Tensor, Epilogue, MatMulAttrs, LinearAttrs, QuantLinearAttrs,
    OK, INVALID_ARGUMENT, UNSUPPORTED, NOT_INITIALIZED, OUT_OF_MEMORY, INTERNAL,
    OUT_S32, OUT_S8, OUT_U8, OUT_F32, OUT_F16, ACT_NONE, ACT_RELU, ACT_GELU,
    ACT_SIGMOID, ACT_TANH, ACT_LEAKY_RELU, ACT_SILU, ACT_HARDSWISH, ACT_ELU, ACT_RELU6,
    DT_F32, DT_F16, DT_S8, DT_U8, DT_S32, DT_Q4_1, BACKEND_HIP, BACKEND_CPU, LAYOUT_DENSE, LAYOUT_PACKED_B_HIP,
    EP_NONE, EP_RELU, EP_GELU, EP_SIGMOID, EP_TANH, EP_LEAKY_RELU, EP_SILU, EP_HARDSWISH, EP_ELU,
    EP_RELU6, EQ_NONE, EQ_REQUANTIZE,
)
from .ops import (  # noqa: F401
    MatMul, Linear, QuantizeLinear, DequantizeLinear, gemm_i8, gemm_q4_1, gemm_fp, tensor, q4_1_quantize, q4_1_dequantize,
)
