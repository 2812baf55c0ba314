// Output pass of the fp x q4_1 routes (nnops_hip_fp_output_pass): the Q4_1
// GEMM writes f32 results into the caller's workspace and this pass adds the
// bias, the residual and the epilogue, or runs the gated combine of Linear's
// gated form, writing the f32 / f16 destination.
//
// Kernel
//   fp_out_pass   one thread per 4 consecutive output columns of a row
//                 (16-byte loads of the f32 results when the row allows),
//                 every float operation a separately rounded one, in the
//                 reference's order. Bound: HBM (rows x n x (4 + 4 or 2)
//                 bytes, twice the source columns when gated).
#include "common.hpp"

namespace nnops_amd {
namespace {

struct FpOut {
    const float* src;
    int64_t ld_src;
    void* out;
    int64_t ld_out;
    int64_t rows;
    int n;
    int out_f16;
    const void* bias;
    EpiParams ep;               // act, act_alpha, act_beta, min_clip, max_clip, out_kind
    int add_to, residual_pre;
    int gated, gate_act;
    float gate_alpha, gate_beta, gate_limit;
    int mm;                     // MatMul's order: alpha P + T(beta old + bias)
    float alpha, beta;
};

__device__ __forceinline__ float round_out(bool f16, float x)
{
    return f16 ? (float)(_Float16)x : x;
}

__device__ __forceinline__ float bias_at(const FpOut& p, int c)
{
    if (p.bias == nullptr) {
        return 0.0f;
    }
    return p.out_f16 ? (float)static_cast<const _Float16*>(p.bias)[c] : static_cast<const float*>(p.bias)[c];
}

// The gate activations of gate_act_scalar (gate_combine.hpp:70-85), with the
// device library's expf / tanhf.
__device__ __forceinline__ float gate_act(const FpOut& p, float g)
{
    switch (p.gate_act) {
    case NNOPS_ACT_SILU:
        return __fdiv_rn(g, __fadd_rn(1.0f, expf(__fmul_rn(-p.gate_alpha, g))));
    case NNOPS_ACT_GELU: {
        const float inner = __fadd_rn(g, __fmul_rn(__fmul_rn(__fmul_rn(0.044715f, g), g), g));
        return __fmul_rn(__fmul_rn(0.5f, g), __fadd_rn(1.0f, tanhf(__fmul_rn(0.7978845608028654f, inner))));
    }
    case NNOPS_ACT_RELU:
        return g > 0.0f ? g : 0.0f;
    case NNOPS_ACT_SIGMOID:
        return __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-g)));
    case NNOPS_ACT_TANH:
        return tanhf(g);
    default:
        return g;
    }
}

__global__ __launch_bounds__(256) void fp_out_pass(FpOut p, int cblocks)
{
    const int64_t r = blockIdx.x / cblocks;
    const int c0 = ((blockIdx.x % cblocks) * 256 + threadIdx.x) * 4;
    if (c0 >= p.n) {
        return;
    }
    const bool f16 = p.out_f16 != 0;
    const float* srow = p.src + r * p.ld_src;
    char* orow = static_cast<char*>(p.out) + r * p.ld_out * (f16 ? 2 : 4);
    const int cn = min(4, p.n - c0);
    // 16-byte loads of the f32 results where the row segment allows
    const bool vec = cn == 4 && (((uintptr_t)(srow + c0)) & 15) == 0 &&
                     (!p.gated || (((uintptr_t)(srow + p.n + c0)) & 15) == 0);
    float a[4], v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (vec) {
        const v4f x = *reinterpret_cast<const v4f*>(srow + c0);
        a[0] = x[0], a[1] = x[1], a[2] = x[2], a[3] = x[3];
        if (p.gated) {
            const v4f y = *reinterpret_cast<const v4f*>(srow + p.n + c0);
            v[0] = y[0], v[1] = y[1], v[2] = y[2], v[3] = y[3];
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            a[e] = e < cn ? srow[c0 + e] : 0.0f;
            if (p.gated) {
                v[e] = e < cn ? srow[p.n + c0 + e] : 0.0f;
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (e >= cn) {
            break;
        }
        const int c = c0 + e;
        float old = 0.0f;
        const float beta = p.residual_pre ? 1.0f : p.beta;
        if (p.mm ? beta != 0.0f : p.add_to) {
            old = f16 ? (float)reinterpret_cast<const _Float16*>(orow)[c] : reinterpret_cast<const float*>(orow)[c];
        }
        float y;
        if (p.mm) {
            // the accumulator init (C primed with beta old + bias, stored in
            // the output type), then the scaled product joins it
            float init = 0.0f;
            if (p.bias != nullptr) {
                init = beta == 0.0f ? bias_at(p, c) : round_out(f16, __fadd_rn(__fmul_rn(old, beta), bias_at(p, c)));
            } else if (beta == 1.0f) {
                init = old;
            } else if (beta != 0.0f) {
                init = round_out(f16, __fmul_rn(old, beta));
            }
            const float prod = p.alpha == 1.0f ? a[e] : __fmul_rn(a[e], p.alpha);
            y = apply_act_fp(p.ep, __fadd_rn(prod, init));
        } else if (p.gated) {
            // the reference's [rows, 2n] tile is of the output's type
            float g = round_out(f16, __fadd_rn(a[e], bias_at(p, c)));
            float u = round_out(f16, __fadd_rn(v[e], bias_at(p, p.n + c)));
            if (__builtin_isfinite(p.gate_limit)) {
                g = fmaxf(fminf(g, p.gate_limit), -p.gate_limit);
                u = fmaxf(fminf(u, p.gate_limit), -p.gate_limit);
            }
            y = apply_act_fp(p.ep, __fmul_rn(gate_act(p, g), __fadd_rn(u, p.gate_beta)));
            if (p.add_to) {
                // the combined value is of the destination's type before it accumulates
                y = __fadd_rn(old, round_out(f16, y));
            }
        } else {
            y = __fadd_rn(a[e], bias_at(p, c));
            if (p.add_to && p.residual_pre) {
                y = __fadd_rn(y, old);
            }
            y = apply_act_fp(p.ep, y);
            if (p.add_to && !p.residual_pre) {
                y = __fadd_rn(round_out(f16, y), old);
            }
        }
        if (f16) {
            reinterpret_cast<_Float16*>(orow)[c] = (_Float16)y;
        } else {
            reinterpret_cast<float*>(orow)[c] = y;
        }
    }
}

bool gate_act_ok(int a)
{
    return a == NNOPS_ACT_NONE || a == NNOPS_ACT_RELU || a == NNOPS_ACT_GELU || a == NNOPS_ACT_SIGMOID ||
           a == NNOPS_ACT_TANH || a == NNOPS_ACT_SILU;
}

}  // namespace
}  // namespace nnops_amd

using namespace nnops_amd;

extern "C" int nnops_hip_fp_output_pass(const NnopsFpOutArgs* a, void* stream)
{
    if (a == nullptr || a->rows < 0 || a->n < 0 || a->n > INT32_MAX) {
        return NNOPS_INVALID_ARGUMENT;
    }
    if (a->rows == 0 || a->n == 0) {
        return NNOPS_OK;
    }
    if (a->src == nullptr || a->out == nullptr || a->ld_src < (a->gated ? 2 : 1) * a->n || a->ld_out < a->n) {
        return NNOPS_INVALID_ARGUMENT;
    }
    if (a->act < NNOPS_ACT_NONE || a->act > NNOPS_ACT_RELU6 || (a->gated && !gate_act_ok(a->gate_act)) ||
        (a->gated && a->add_to && a->residual_pre) || (a->gated && a->matmul_order)) {
        return NNOPS_UNSUPPORTED;
    }
    FpOut p{};
    p.src = a->src;
    p.ld_src = a->ld_src;
    p.out = a->out;
    p.ld_out = a->ld_out;
    p.rows = a->rows;
    p.n = (int)a->n;
    p.out_f16 = a->out_f16 != 0;
    p.bias = a->bias;
    p.ep.act = a->act;
    p.ep.act_alpha = a->act_alpha;
    p.ep.act_beta = a->act_beta;
    p.ep.min_clip = a->min_clip;
    p.ep.max_clip = a->max_clip;
    p.ep.out_kind = p.out_f16 ? NNOPS_OUT_F16 : NNOPS_OUT_F32;
    p.add_to = a->add_to != 0;
    p.residual_pre = a->residual_pre != 0;
    p.gated = a->gated != 0;
    p.gate_act = a->gate_act;
    p.gate_alpha = a->gate_alpha;
    p.gate_beta = a->gate_beta;
    p.gate_limit = a->gate_limit;
    p.mm = a->matmul_order != 0;
    p.alpha = a->alpha;
    p.beta = a->beta;
    const int64_t cblocks = (a->n + 1023) / 1024;
    if (cblocks * a->rows > INT32_MAX) {
        return NNOPS_UNSUPPORTED;
    }
    hipLaunchKernelGGL(fp_out_pass, dim3((unsigned)(cblocks * a->rows)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), p, (int)cblocks);
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}
