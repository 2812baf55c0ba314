// The fp x q4_1 routes' output pass as device functions: bias, residual,
// epilogue, or the gated combine of Linear's gated form, over one f32 product
// (two for the gated form), in the reference's order, every float operation a
// separately rounded one. Shared by fp_out_pass (a pass over a staged f32
// product) and the Q4_1 ring GEMM's fused write-back.
#pragma once

#include "common.hpp"

namespace nnops_amd {

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

// Checks the arguments and fills the device form (NNOPS_OK or the status).
int make_fp_out(const NnopsFpOutArgs* a, FpOut& p);

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

// Whether the destination's current value takes part.
__device__ __forceinline__ bool fp_out_reads_old(const FpOut& p)
{
    const float beta = p.residual_pre ? 1.0f : p.beta;
    return p.mm ? beta != 0.0f : p.add_to != 0;
}

__device__ __forceinline__ float fp_out_old(const FpOut& p, const char* orow, int c)
{
    if (!fp_out_reads_old(p)) {
        return 0.0f;
    }
    return p.out_f16 ? (float)reinterpret_cast<const _Float16*>(orow)[c] : reinterpret_cast<const float*>(orow)[c];
}

// A destination element from the product a (and, gated, the value half's
// product v), the destination's current value `old` (fp_out_old) and the
// bias values of its column (bg = bias_at(c); gated, bu = bias_at(n + c)):
// the value to store, in f32 (rounded to f16 by the store when out_f16).
__device__ __forceinline__ float fp_out_value(const FpOut& p, float a, float v, float old, float bg, float bu)
{
    const bool f16 = p.out_f16 != 0;
    const float beta = p.residual_pre ? 1.0f : p.beta;
    float y;
    if (p.mm) {
        // the accumulator init (C primed with beta old + bias, stored in
        // the output type), then the scaled product joins it
        float init = 0.0f;
        if (p.bias != nullptr) {
            init = beta == 0.0f ? bg : round_out(f16, __fadd_rn(__fmul_rn(old, beta), bg));
        } else if (beta == 1.0f) {
            init = old;
        } else if (beta != 0.0f) {
            init = round_out(f16, __fmul_rn(old, beta));
        }
        const float prod = p.alpha == 1.0f ? a : __fmul_rn(a, p.alpha);
        y = apply_act_fp(p.ep, __fadd_rn(prod, init));
    } else if (p.gated) {
        // the reference's [rows, 2n] tile is of the output's type
        float g = round_out(f16, __fadd_rn(a, bg));
        float u = round_out(f16, __fadd_rn(v, bu));
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
        y = __fadd_rn(a, bg);
        if (p.add_to && p.residual_pre) {
            y = __fadd_rn(y, old);
        }
        y = apply_act_fp(p.ep, y);
        if (p.add_to && !p.residual_pre) {
            y = __fadd_rn(round_out(f16, y), old);
        }
    }
    return y;
}

__device__ __forceinline__ void fp_out_store(const FpOut& p, char* orow, int c, float y)
{
    if (p.out_f16) {
        reinterpret_cast<_Float16*>(orow)[c] = (_Float16)y;
    } else {
        reinterpret_cast<float*>(orow)[c] = y;
    }
}

}  // namespace nnops_amd
