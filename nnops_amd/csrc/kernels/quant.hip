// QuantizeLinear / DequantizeLinear on gfx950: the elementwise steps either
// side of the int8 GEMM in a QDQ graph, and the activation quantization of
// the fp-activation int8 MatMul. One thread per 4 consecutive elements of a
// rows x cols view (row strides in elements); the parameter of flat element
// i = r * cols + c is entry (i / inner) % dim of the scale / zero-point
// tables (per tensor: dim = 1; per token: inner = cols; per channel: the
// axis decomposition). Bound: HBM.
//
// Rounding and order follow nnops' x86 kernels bit for bit
// (src/backend/cpu/x86_64/quant.hpp):
//   quantize    q = clamp(rint(fma(x, 1 / s, zp)), qmin, qmax), ties to even;
//               a NaN or |v| >= 2^31 converts to the integer indefinite, so it
//               saturates to qmin;
//   dequantize  y = fma(q, s, -zp * s) over each segment's whole 16-element
//               blocks (the vector body) and (q - zp) * s over its last
//               segment % 16 elements (the scalar tail). The segment is the
//               reference's row: numel per tensor, cols per token, inner per
//               channel.
#include "common.hpp"

namespace nnops_amd {
namespace {

struct QdqKern {
    const void* x;
    void* y;
    int64_t rows, cols, ld_x, ld_y;
    int32_t x_kind, y_kind, zp_kind;
    const float* scale;
    const void* zero_point;
    float scale_scalar;
    int32_t zp_scalar;
    int64_t inner, dim, segment;
};

__device__ __forceinline__ int64_t qdq_param(const QdqKern& p, int64_t i)
{
    return p.dim <= 1 ? 0 : (i / p.inner) % p.dim;
}

__device__ __forceinline__ float qdq_scale(const QdqKern& p, int64_t j)
{
    return p.scale != nullptr ? p.scale[j] : p.scale_scalar;
}

__device__ __forceinline__ int32_t qdq_zero(const QdqKern& p, int64_t j)
{
    if (p.zero_point == nullptr) {
        return p.zp_scalar;
    }
    switch (p.zp_kind) {
    case NNOPS_OUT_S8: return static_cast<const int8_t*>(p.zero_point)[j];
    case NNOPS_OUT_U8: return static_cast<const uint8_t*>(p.zero_point)[j];
    default: return static_cast<const int32_t*>(p.zero_point)[j];
    }
}

__global__ __launch_bounds__(256) void quantize_kernel(QdqKern p)
{
    const int64_t groups = (p.cols + 3) / 4;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= p.rows * groups) {
        return;
    }
    const int64_t r = t / groups, c0 = (t - r * groups) * 4;
    const bool u8 = p.y_kind == NNOPS_OUT_U8;
    const int32_t qmin = u8 ? 0 : -128, qmax = u8 ? 255 : 127;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int64_t c = c0 + e;
        if (c >= p.cols) {
            break;
        }
        const int64_t xi = r * p.ld_x + c;
        const float x = p.x_kind == NNOPS_OUT_F16 ? (float)static_cast<const _Float16*>(p.x)[xi]
                                                  : static_cast<const float*>(p.x)[xi];
        const int64_t j = qdq_param(p, r * p.cols + c);
        const float inv = __fdiv_rn(1.0f, qdq_scale(p, j));
        const float v = __builtin_fmaf(x, inv, (float)qdq_zero(p, j));
        int32_t q = qmin;
        if (__builtin_fabsf(v) < 2147483648.0f) {   // false for NaN
            q = (int32_t)__builtin_rintf(v);
            q = q < qmin ? qmin : (q > qmax ? qmax : q);
        }
        const int64_t yi = r * p.ld_y + c;
        if (u8) {
            static_cast<uint8_t*>(p.y)[yi] = (uint8_t)q;
        } else {
            static_cast<int8_t*>(p.y)[yi] = (int8_t)q;
        }
    }
}

__global__ __launch_bounds__(256) void dequantize_kernel(QdqKern p)
{
    const int64_t groups = (p.cols + 3) / 4;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= p.rows * groups) {
        return;
    }
    const int64_t r = t / groups, c0 = (t - r * groups) * 4;
    const int64_t body = p.segment - p.segment % 16;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int64_t c = c0 + e;
        if (c >= p.cols) {
            break;
        }
        const int64_t xi = r * p.ld_x + c;
        const int32_t q = p.x_kind == NNOPS_OUT_U8 ? (int32_t) static_cast<const uint8_t*>(p.x)[xi]
                                                   : (int32_t) static_cast<const int8_t*>(p.x)[xi];
        const int64_t i = r * p.cols + c;
        const int64_t j = qdq_param(p, i);
        const float s = qdq_scale(p, j);
        const float zf = (float)qdq_zero(p, j);
        float y;
        if (i % p.segment < body) {
            y = __builtin_fmaf((float)q, s, __fmul_rn(-zf, s));
        } else {
            y = __fmul_rn(__fsub_rn((float)q, zf), s);
        }
        const int64_t yi = r * p.ld_y + c;
        if (p.y_kind == NNOPS_OUT_F16) {
            static_cast<_Float16*>(p.y)[yi] = (_Float16)y;
        } else {
            static_cast<float*>(p.y)[yi] = y;
        }
    }
}

int qdq_check(const NnopsQdqArgs* g, bool quantize)
{
    if (g == nullptr || g->rows < 0 || g->cols < 0) {
        return NNOPS_INVALID_ARGUMENT;
    }
    if (g->rows == 0 || g->cols == 0) {
        return NNOPS_OK;
    }
    if (g->x == nullptr || g->y == nullptr || g->ld_x < g->cols || g->ld_y < g->cols ||
        (g->dim > 1 && g->inner <= 0) || g->dim < 0 || (g->scale == nullptr && !(g->scale_scalar != 0.0f))) {
        return NNOPS_INVALID_ARGUMENT;
    }
    const bool fx = g->x_kind == NNOPS_OUT_F32 || g->x_kind == NNOPS_OUT_F16;
    const bool iy = g->y_kind == NNOPS_OUT_S8 || g->y_kind == NNOPS_OUT_U8;
    const bool ix = g->x_kind == NNOPS_OUT_S8 || g->x_kind == NNOPS_OUT_U8;
    const bool fy = g->y_kind == NNOPS_OUT_F32 || g->y_kind == NNOPS_OUT_F16;
    if (quantize ? !(fx && iy) : !(ix && fy)) {
        return NNOPS_UNSUPPORTED;
    }
    if (!quantize && g->segment <= 0) {
        return NNOPS_INVALID_ARGUMENT;
    }
    return -1;
}

QdqKern qdq_kern(const NnopsQdqArgs* g)
{
    QdqKern k{};
    k.x = g->x;
    k.y = g->y;
    k.rows = g->rows;
    k.cols = g->cols;
    k.ld_x = g->ld_x;
    k.ld_y = g->ld_y;
    k.x_kind = g->x_kind;
    k.y_kind = g->y_kind;
    k.zp_kind = g->zp_kind;
    k.scale = g->scale;
    k.zero_point = g->zero_point;
    k.scale_scalar = g->scale_scalar;
    k.zp_scalar = g->zp_scalar;
    k.inner = g->inner;
    k.dim = g->dim;
    k.segment = g->segment;
    return k;
}

}  // namespace
}  // namespace nnops_amd

using namespace nnops_amd;

extern "C" int nnops_hip_quantize_linear(const NnopsQdqArgs* g, void* stream)
{
    const int rc = qdq_check(g, true);
    if (rc >= 0) {
        return rc;
    }
    const int64_t threads = g->rows * ((g->cols + 3) / 4);
    hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), qdq_kern(g));
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}

extern "C" int nnops_hip_dequantize_linear(const NnopsQdqArgs* g, void* stream)
{
    const int rc = qdq_check(g, false);
    if (rc >= 0) {
        return rc;
    }
    const int64_t threads = g->rows * ((g->cols + 3) / 4);
    hipLaunchKernelGGL(dequantize_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), qdq_kern(g));
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}
