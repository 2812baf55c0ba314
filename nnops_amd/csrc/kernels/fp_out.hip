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
#include "fp_out.hpp"

namespace nnops_amd {
namespace {

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
        const float y = fp_out_value(p, a[e], v[e], fp_out_old(p, orow, c), bias_at(p, c),
                                     p.gated ? bias_at(p, p.n + c) : 0.0f);
        fp_out_store(p, orow, c, y);
    }
}

bool gate_act_ok(int a)
{
    return a == NNOPS_ACT_NONE || a == NNOPS_ACT_RELU || a == NNOPS_ACT_GELU || a == NNOPS_ACT_SIGMOID ||
           a == NNOPS_ACT_TANH || a == NNOPS_ACT_SILU;
}

}  // namespace

int make_fp_out(const NnopsFpOutArgs* a, FpOut& p)
{
    if (a == nullptr || a->rows < 0 || a->n < 0 || a->n > INT32_MAX) {
        return NNOPS_INVALID_ARGUMENT;
    }
    if (a->out == nullptr || a->ld_out < a->n) {
        return NNOPS_INVALID_ARGUMENT;
    }
    if (a->act < NNOPS_ACT_NONE || a->act > NNOPS_ACT_RELU6 || (a->gated && !gate_act_ok(a->gate_act)) ||
        (a->gated && a->add_to && a->residual_pre) || (a->gated && a->matmul_order)) {
        return NNOPS_UNSUPPORTED;
    }
    p = FpOut{};
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
    return NNOPS_OK;
}

}  // namespace nnops_amd

using namespace nnops_amd;

extern "C" int nnops_hip_fp_output_pass(const NnopsFpOutArgs* a, void* stream)
{
    const TimingDisarm disarm;
    if (a == nullptr || a->rows < 0 || a->n < 0 || a->n > INT32_MAX) {
        return NNOPS_INVALID_ARGUMENT;
    }
    if (a->rows == 0 || a->n == 0) {
        return NNOPS_OK;
    }
    if (a->src == nullptr || a->ld_src < (a->gated ? 2 : 1) * a->n) {
        return NNOPS_INVALID_ARGUMENT;
    }
    FpOut p;
    if (const int rc = make_fp_out(a, p); rc != NNOPS_OK) {
        return rc;
    }
    const int64_t cblocks = (a->n + 1023) / 1024;
    if (cblocks * a->rows > INT32_MAX) {
        return NNOPS_UNSUPPORTED;
    }
    NNOPS_LAUNCH(fp_out_pass, dim3((unsigned)(cblocks * a->rows)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), p, (int)cblocks);
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}
