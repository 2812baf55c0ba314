// QuantizeLinear / DequantizeLinear on gfx950: the elementwise steps either
// side of the int8 GEMM in a QDQ graph, and the activation quantization of
// the fp-activation int8 MatMul. One thread per 16 consecutive elements of a
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

// The parameter of element (r, c) of the rows x cols view, without a 64-bit
// division for per-tensor (dim <= 1) and per-token (inner == cols,
// dim == rows) tables.
__device__ __forceinline__ int64_t qdq_param_rc(const QdqKern& p, int64_t r, int64_t c)
{
    if (p.dim <= 1) {
        return 0;
    }
    if (p.inner == p.cols && p.dim == p.rows) {
        return r;
    }
    return qdq_param(p, r * p.cols + c);
}

// Does the 16-element chunk at (r, c0) share one parameter?
__device__ __forceinline__ bool qdq_uniform_rc(const QdqKern& p, int64_t r, int64_t c0)
{
    if (p.dim <= 1 || (p.inner == p.cols && p.dim == p.rows)) {
        return true;                              // one parameter per row (or per tensor)
    }
    const int64_t i = r * p.cols + c0;
    return (i / p.inner) == ((i + 15) / p.inner);
}

// Chunk t of the launch -> (row, first column), in 32-bit arithmetic when the
// chunk count allows it.
__device__ __forceinline__ void qdq_chunk(const QdqKern& p, int64_t t, int64_t chunks, int64_t& r, int64_t& c0)
{
    if (p.rows * chunks <= (int64_t)UINT32_MAX) {
        const uint32_t tt = (uint32_t)t, ch = (uint32_t)chunks;
        const uint32_t rr = tt / ch;
        r = rr;
        c0 = (int64_t)(tt - rr * ch) * 16;
    } else {
        r = t / chunks;
        c0 = (t - r * chunks) * 16;
    }
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

__device__ __forceinline__ float qdq_load_x(const QdqKern& p, int64_t xi)
{
    return p.x_kind == NNOPS_OUT_F16 ? (float)static_cast<const _Float16*>(p.x)[xi]
                                     : static_cast<const float*>(p.x)[xi];
}

__device__ __forceinline__ int32_t quant_one(float x, float inv, float zf, int32_t qmin, int32_t qmax)
{
    const float v = __builtin_fmaf(x, inv, zf);
    int32_t q = qmin;
    if (__builtin_fabsf(v) < 2147483648.0f) {   // false for NaN
        q = (int32_t)__builtin_rintf(v);
        q = q < qmin ? qmin : (q > qmax ? qmax : q);
    }
    return q;
}


// One thread per 16 consecutive elements of a row (a chunk): 16-byte vector
// loads and stores when the chunk is whole, aligned and under one parameter
// (every per-tensor and per-token case with 16 | cols, per-channel with
// 16 | inner), element by element otherwise.
__global__ __launch_bounds__(256) void quantize_kernel(QdqKern p)
{
    const int64_t chunks = (p.cols + 15) / 16;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= p.rows * chunks) {
        return;
    }
    int64_t r, c0;
    qdq_chunk(p, t, chunks, r, c0);
    const bool u8 = p.y_kind == NNOPS_OUT_U8;
    const int32_t qmin = u8 ? 0 : -128, qmax = u8 ? 255 : 127;
    const int64_t i0 = r * p.cols + c0;
    const int64_t xi = r * p.ld_x + c0, yi = r * p.ld_y + c0;
    const bool f16 = p.x_kind == NNOPS_OUT_F16;
    const bool vec = c0 + 16 <= p.cols && qdq_uniform_rc(p, r, c0) &&
                     ((uintptr_t)p.x + (uintptr_t)xi * (f16 ? 2 : 4)) % 16 == 0 &&
                     ((uintptr_t)p.y + (uintptr_t)yi) % 16 == 0;
    if (vec) {
        const int64_t j = qdq_param_rc(p, r, c0);
        const float inv = __fdiv_rn(1.0f, qdq_scale(p, j));
        const float zf = (float)qdq_zero(p, j);
        float x[16];
        if (f16) {
            const v4i* src = reinterpret_cast<const v4i*>(static_cast<const _Float16*>(p.x) + xi);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const v4i w = __builtin_nontemporal_load(src + h);
                const _Float16* e = reinterpret_cast<const _Float16*>(&w);
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    x[8 * h + q] = (float)e[q];
                }
            }
        } else {
            const v4i* src = reinterpret_cast<const v4i*>(static_cast<const float*>(p.x) + xi);
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const v4i w = __builtin_nontemporal_load(src + h);
                x[4 * h + 0] = __int_as_float(w.x);
                x[4 * h + 1] = __int_as_float(w.y);
                x[4 * h + 2] = __int_as_float(w.z);
                x[4 * h + 3] = __int_as_float(w.w);
            }
        }
        uint32_t o[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            o[e / 4] |= ((uint32_t)quant_one(x[e], inv, zf, qmin, qmax) & 0xffu) << (8 * (e % 4));
        }
        __builtin_nontemporal_store(v4i{(int)o[0], (int)o[1], (int)o[2], (int)o[3]},
                                    reinterpret_cast<v4i*>(static_cast<int8_t*>(p.y) + yi));
        return;
    }
    for (int e = 0; e < 16 && c0 + e < p.cols; ++e) {
        const int64_t j = qdq_param(p, i0 + e);
        const float inv = __fdiv_rn(1.0f, qdq_scale(p, j));
        const int32_t q = quant_one(qdq_load_x(p, xi + e), inv, (float)qdq_zero(p, j), qmin, qmax);
        if (u8) {
            static_cast<uint8_t*>(p.y)[yi + e] = (uint8_t)q;
        } else {
            static_cast<int8_t*>(p.y)[yi + e] = (int8_t)q;
        }
    }
}

// The common shape, an f16 side and one parameter per row (per tensor or per
// token) with 1024 | cols and 16-byte aligned rows: a wave owns 1024
// consecutive elements of one row and lane l the elements 8 l .. 8 l + 7 and
// 512 + 8 l .. + 7, so every vector load and store instruction of the wave
// covers one contiguous span (1 KiB of f16, 512 bytes of int8), where the
// general kernels' 16-element chunks per lane touch each line twice, half of
// it per instruction. The same operations per element as quant_one /
// dequantize's vector body (fma(q, s, -zp * s): 16 | cols makes every element
// a body element).
__host__ __device__ __forceinline__ bool qdq_row_param(const QdqKern& p)
{
    return p.dim <= 1 || (p.inner == p.cols && p.dim == p.rows);
}

__global__ __launch_bounds__(256) void quantize_rows_f16(QdqKern p)
{
    const int lane = threadIdx.x & 63;
    const int64_t wblk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t per_row = p.cols / 1024;
    if (wblk >= p.rows * per_row) {
        return;
    }
    const int64_t r = wblk / per_row;
    const int64_t c0 = (wblk - r * per_row) * 1024;
    const int64_t j = p.dim <= 1 ? 0 : r;
    const float inv = __fdiv_rn(1.0f, qdq_scale(p, j));
    const float zf = (float)qdq_zero(p, j);
    const bool u8 = p.y_kind == NNOPS_OUT_U8;
    const int32_t qmin = u8 ? 0 : -128, qmax = u8 ? 255 : 127;
    const _Float16* xr = static_cast<const _Float16*>(p.x) + r * p.ld_x + c0;
    int8_t* yr = static_cast<int8_t*>(p.y) + r * p.ld_y + c0;
    v4i w[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        w[h] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(xr + 512 * h + 8 * lane));
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const _Float16* e = reinterpret_cast<const _Float16*>(&w[h]);
        uint32_t o[2] = {0u, 0u};
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            o[q / 4] |= ((uint32_t)quant_one((float)e[q], inv, zf, qmin, qmax) & 0xffu) << (8 * (q % 4));
        }
        __builtin_nontemporal_store((uint64_t)o[0] | ((uint64_t)o[1] << 32),
                                    reinterpret_cast<uint64_t*>(yr + 512 * h + 8 * lane));
    }
}

__global__ __launch_bounds__(256) void dequantize_rows_f16(QdqKern p)
{
    const int lane = threadIdx.x & 63;
    const int64_t wblk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t per_row = p.cols / 1024;
    if (wblk >= p.rows * per_row) {
        return;
    }
    const int64_t r = wblk / per_row;
    const int64_t c0 = (wblk - r * per_row) * 1024;
    const int64_t j = p.dim <= 1 ? 0 : r;
    const float sc = qdq_scale(p, j);
    const float zf = (float)qdq_zero(p, j);
    const float nzs = __fmul_rn(-zf, sc);
    const bool u8 = p.x_kind == NNOPS_OUT_U8;
    const int8_t* xr = static_cast<const int8_t*>(p.x) + r * p.ld_x + c0;
    _Float16* yr = static_cast<_Float16*>(p.y) + r * p.ld_y + c0;
    uint64_t w[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        w[h] = __builtin_nontemporal_load(reinterpret_cast<const uint64_t*>(xr + 512 * h + 8 * lane));
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        _Float16 e8[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t b = (uint32_t)(w[h] >> (8 * q)) & 0xffu;
            const int32_t v = u8 ? (int32_t)b : (int32_t)(int8_t)b;
            // the f32 result first, then its f16 rounding (two roundings, as
            // the reference): the asm keeps the compiler from fusing the pair
            // into one mixed-precision fma that rounds once
            float f = __builtin_fmaf((float)v, sc, nzs);
            asm volatile("" : "+v"(f));
            e8[q] = (_Float16)f;
        }
        v4i o;
        __builtin_memcpy(&o, e8, 16);
        __builtin_nontemporal_store(o, reinterpret_cast<v4i*>(yr + 512 * h + 8 * lane));
    }
}

// fma(q, s, -zp * s) over each segment's whole 16-element blocks, (q - zp) * s
// over its last segment % 16 elements.
__device__ __forceinline__ float dequant_one(const QdqKern& p, int64_t i, int32_t q, float s, float zf)
{
    const int64_t body = p.segment - p.segment % 16;
    if (i % p.segment < body) {
        return __builtin_fmaf((float)q, s, __fmul_rn(-zf, s));
    }
    return __fmul_rn(__fsub_rn((float)q, zf), s);
}

__global__ __launch_bounds__(256) void dequantize_kernel(QdqKern p)
{
    const int64_t chunks = (p.cols + 15) / 16;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= p.rows * chunks) {
        return;
    }
    int64_t r, c0;
    qdq_chunk(p, t, chunks, r, c0);
    const int64_t i0 = r * p.cols + c0;
    const int64_t xi = r * p.ld_x + c0, yi = r * p.ld_y + c0;
    const bool f16 = p.y_kind == NNOPS_OUT_F16;
    const bool u8 = p.x_kind == NNOPS_OUT_U8;
    const int64_t body = p.segment - p.segment % 16;
    // whole chunk inside one segment's vector body (or wholly in its tail);
    // per token the segment is the row, per tensor the whole view
    const int64_t s0 = p.segment == p.cols ? c0 : (p.segment == p.rows * p.cols ? i0 : i0 % p.segment);
    const bool one_form = s0 + 15 < p.segment && ((s0 < body) == (s0 + 15 < body));
    const bool vec = c0 + 16 <= p.cols && qdq_uniform_rc(p, r, c0) && one_form &&
                     ((uintptr_t)p.x + (uintptr_t)xi) % 16 == 0 &&
                     ((uintptr_t)p.y + (uintptr_t)yi * (f16 ? 2 : 4)) % 16 == 0;
    if (vec) {
        const int64_t j = qdq_param_rc(p, r, c0);
        const float sc = qdq_scale(p, j);
        const float zf = (float)qdq_zero(p, j);
        const bool fused = s0 < body;
        const float nzs = __fmul_rn(-zf, sc);
        const v4i w = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(static_cast<const int8_t*>(p.x) + xi));
        const uint32_t wd[4] = {(uint32_t)w.x, (uint32_t)w.y, (uint32_t)w.z, (uint32_t)w.w};
        float y[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t b = (wd[e / 4] >> (8 * (e % 4))) & 0xffu;
            const int32_t q = u8 ? (int32_t)b : (int32_t)(int8_t)b;
            y[e] = fused ? __builtin_fmaf((float)q, sc, nzs) : __fmul_rn(__fsub_rn((float)q, zf), sc);
        }
        if (f16) {
            v4i* dst = reinterpret_cast<v4i*>(static_cast<_Float16*>(p.y) + yi);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                _Float16 e8[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    float f = y[8 * h + q];
                    asm volatile("" : "+v"(f));   // f32 first, then f16 (see dequantize_rows_f16)
                    e8[q] = (_Float16)f;
                }
                v4i o;
                __builtin_memcpy(&o, e8, 16);
                __builtin_nontemporal_store(o, dst + h);
            }
        } else {
            v4i* dst = reinterpret_cast<v4i*>(static_cast<float*>(p.y) + yi);
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                __builtin_nontemporal_store(v4i{__float_as_int(y[4 * h]), __float_as_int(y[4 * h + 1]),
                                                 __float_as_int(y[4 * h + 2]), __float_as_int(y[4 * h + 3])},
                                            dst + h);
            }
        }
        return;
    }
    for (int e = 0; e < 16 && c0 + e < p.cols; ++e) {
        const int32_t q = u8 ? (int32_t) static_cast<const uint8_t*>(p.x)[xi + e]
                             : (int32_t) static_cast<const int8_t*>(p.x)[xi + e];
        const int64_t j = qdq_param(p, i0 + e);
        const float y = dequant_one(p, i0 + e, q, qdq_scale(p, j), (float)qdq_zero(p, j));
        if (f16) {
            static_cast<_Float16*>(p.y)[yi + e] = (_Float16)y;
        } else {
            static_cast<float*>(p.y)[yi + e] = y;
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

// The rows kernels' conditions: the f16 side, one parameter per row, 1024 |
// cols, 16-byte aligned f16 rows and 8-byte aligned int8 rows, and for the
// dequantize the segment a multiple of 16 (every element in a vector body).
bool rows_fast(const QdqKern& k, bool quantize)
{
    const bool f16 = quantize ? k.x_kind == NNOPS_OUT_F16 : k.y_kind == NNOPS_OUT_F16;
    const void* h = quantize ? k.x : k.y;
    const void* b = quantize ? k.y : k.x;
    const int64_t ldh = quantize ? k.ld_x : k.ld_y, ldb = quantize ? k.ld_y : k.ld_x;
    return f16 && qdq_row_param(k) && k.cols % 1024 == 0 && k.cols > 0 && ((uintptr_t)h % 16) == 0 &&
           (ldh * 2) % 16 == 0 && ((uintptr_t)b % 8) == 0 && ldb % 8 == 0 &&
           (quantize || k.segment % 16 == 0) && k.rows * (k.cols / 1024) <= 4 * (int64_t)UINT32_MAX;
}

}  // namespace
}  // namespace nnops_amd

using namespace nnops_amd;

extern "C" int nnops_hip_quantize_linear(const NnopsQdqArgs* g, void* stream)
{
    const TimingDisarm disarm;
    const int rc = qdq_check(g, true);
    if (rc >= 0) {
        return rc;
    }
    const QdqKern k = qdq_kern(g);
    if (rows_fast(k, true)) {
        const int64_t waves = g->rows * (g->cols / 1024);
        NNOPS_LAUNCH(quantize_rows_f16, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), k);
        return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
    }
    const int64_t threads = g->rows * ((g->cols + 15) / 16);
    NNOPS_LAUNCH(quantize_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), k);
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}

extern "C" int nnops_hip_dequantize_linear(const NnopsQdqArgs* g, void* stream)
{
    const TimingDisarm disarm;
    const int rc = qdq_check(g, false);
    if (rc >= 0) {
        return rc;
    }
    const QdqKern k = qdq_kern(g);
    if (rows_fast(k, false)) {
        const int64_t waves = g->rows * (g->cols / 1024);
        NNOPS_LAUNCH(dequantize_rows_f16, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), k);
        return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
    }
    const int64_t threads = g->rows * ((g->cols + 15) / 16);
    NNOPS_LAUNCH(dequantize_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), k);
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}
