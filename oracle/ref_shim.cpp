// C entry points over the reference's own oracles, so Python tests can call
// them through ctypes. Test infrastructure only: compiled by oracle/Makefile
// (target `ref`) against the nnops sources where they lie, into oracle/_ref/.
// Nothing from the reference is copied here; this file only constructs the
// reference's TensorViews and calls:
//   nnops::backend::cpu::reference::matmul_int8_ref  tests/reference/matmul_int8_ref.cpp:206
//   nnops::backend::cpu::reference::matmul_dq_ref    tests/reference/matmul_dq_ref.cpp:249
//   nnops::quantize_q4 / nnops::pack_q4              include/nnops/detail/q4_1.hpp:92,155
//   nnops::apply_epilogue (Gelu)                     src/backend/cpu/simd_kernel/simd_epilogue.hpp:56
//   nnops::backend::cpu::matmul_int8_requant         simd_epilogue.hpp:137
//   float_to_half / half_to_float                    include/nnops/detail/half.hpp:69-134
#include "nnops/ops/matmul.hpp"
#include "nnops/detail/q4_1.hpp"
#include "simd_kernel/simd_epilogue.hpp"

#include <cstdint>
#include <span>

namespace nnops::backend::cpu::reference {
void matmul_int8_ref(const MatMulAttributes& attrs, TensorView& output,
                     std::span<const TensorView> inputs, const ComputeContext& ctx,
                     void* workspace);
void matmul_dq_ref(const MatMulAttributes& attrs, TensorView& output,
                   std::span<const TensorView> inputs, const ComputeContext& ctx, void* workspace);
}

using namespace nnops;

extern "C" {

// out_kind: 0 s32, 1 s8, 2 u8. Per-token/per-channel arrays may be null.
void ref_matmul_int8(const void* a, const int8_t* b, const int32_t* bias, void* c,
                     int64_t M, int64_t N, int64_t K, int64_t lda_bytes,
                     int64_t ldb_bytes, int64_t ldc_bytes, int trans_b, int a_u8,
                     const float* s_a, float s_a_scalar, const int32_t* zp_a,
                     int32_t zp_a_scalar, const float* s_b, float s_b_scalar,
                     const int32_t* zp_b, int32_t zp_b_scalar, float s_out,
                     int32_t zp_out, int out_kind, int relu)
{
    QuantParams qa;
    qa.granularity = s_a || zp_a ? QuantGranularity::PerToken : QuantGranularity::PerTensor;
    qa.scale = s_a_scalar;
    qa.zero_point = zp_a_scalar;
    qa.scale_data = s_a;
    qa.zero_point_data = zp_a;
    qa.num_scales = (s_a || zp_a) ? M : 0;

    QuantParams qb;
    qb.granularity = s_b || zp_b ? QuantGranularity::PerChannel : QuantGranularity::PerTensor;
    qb.scale = s_b_scalar;
    qb.zero_point = zp_b_scalar;
    qb.scale_data = s_b;
    qb.zero_point_data = zp_b;
    qb.num_scales = (s_b || zp_b) ? N : 0;

    QuantParams qc;
    qc.scale = s_out;
    qc.zero_point = zp_out;

    const int64_t ashape[] = {M, K};
    const int64_t bshape_nn[] = {K, N};
    const int64_t bshape_nt[] = {N, K};
    const int64_t cshape[] = {M, N};
    const int64_t bias_shape[] = {N};

    TensorView av(ashape, a_u8 ? DataType::u8 : DataType::s8, const_cast<void*>(a), lda_bytes,
                  TensorLayout::Dense, qa);
    TensorView bv(trans_b ? std::span<const int64_t>(bshape_nt) : std::span<const int64_t>(bshape_nn),
                  DataType::s8, const_cast<int8_t*>(b), ldb_bytes, TensorLayout::Dense, qb);
    const DataType odt = out_kind == 0 ? DataType::s32 : (out_kind == 1 ? DataType::s8 : DataType::u8);
    TensorView cv(cshape, odt, c, ldc_bytes, TensorLayout::Dense, qc);
    TensorView biasv(bias_shape, DataType::s32, const_cast<int32_t*>(bias));

    MatMulAttributes attrs{};
    attrs.transpose_b = trans_b != 0;
    attrs.output_dtype = odt;
    if (relu) {
        attrs.epilogue.type = EpilogueActivateType::Relu;
    }
    const TensorView ins3[] = {av, bv, biasv};
    ComputeContext ctx{};
    backend::cpu::reference::matmul_int8_ref(
        attrs, cv, std::span<const TensorView>(ins3, bias ? 3 : 2), ctx, nullptr);
}

// fp A (f32, or f16 when a_f16) with per-tensor / per-token QuantParams x s8 B
// -> C in A's dtype; bias (A's dtype, [N]) optional. act: EpilogueActivateType.
void ref_matmul_dq(const void* a, int a_f16, const int8_t* b, const void* bias, void* c,
                   int64_t M, int64_t N, int64_t K, int64_t lda_bytes, int64_t ldb_bytes,
                   int64_t ldc_bytes, int trans_b, int act_u8,
                   const float* s_a, float s_a_scalar, const int32_t* zp_a, int32_t zp_a_scalar,
                   const float* s_b, float s_b_scalar, const int32_t* zp_b, int32_t zp_b_scalar,
                   int act, float alpha, float beta, float min_clip, float max_clip)
{
    QuantParams qa;
    qa.granularity = s_a || zp_a ? QuantGranularity::PerToken : QuantGranularity::PerTensor;
    qa.scale = s_a_scalar;
    qa.zero_point = zp_a_scalar;
    qa.scale_data = s_a;
    qa.zero_point_data = zp_a;
    qa.num_scales = (s_a || zp_a) ? M : 0;

    QuantParams qb;
    qb.granularity = s_b || zp_b ? QuantGranularity::PerChannel : QuantGranularity::PerTensor;
    qb.scale = s_b_scalar;
    qb.zero_point = zp_b_scalar;
    qb.scale_data = s_b;
    qb.zero_point_data = zp_b;
    qb.num_scales = (s_b || zp_b) ? N : 0;

    const int64_t ashape[] = {M, K};
    const int64_t bshape_nn[] = {K, N};
    const int64_t bshape_nt[] = {N, K};
    const int64_t cshape[] = {M, N};
    const int64_t bias_shape[] = {N};
    const DataType fdt = a_f16 ? DataType::f16 : DataType::f32;

    TensorView av(ashape, fdt, const_cast<void*>(a), lda_bytes, TensorLayout::Dense, qa);
    TensorView bv(trans_b ? std::span<const int64_t>(bshape_nt) : std::span<const int64_t>(bshape_nn),
                  DataType::s8, const_cast<int8_t*>(b), ldb_bytes, TensorLayout::Dense, qb);
    TensorView cv(cshape, fdt, c, ldc_bytes);
    TensorView biasv(bias_shape, fdt, const_cast<void*>(bias));

    MatMulAttributes attrs{};
    attrs.transpose_b = trans_b != 0;
    attrs.output_dtype = fdt;
    attrs.act_quant_dtype = act_u8 ? DataType::u8 : DataType::s8;
    attrs.epilogue.type = static_cast<EpilogueActivateType>(act);
    attrs.epilogue.alpha = alpha;
    attrs.epilogue.beta = beta;
    attrs.epilogue.min_clip = min_clip;
    attrs.epilogue.max_clip = max_clip;
    const TensorView ins3[] = {av, bv, biasv};
    ComputeContext ctx{};
    backend::cpu::reference::matmul_dq_ref(
        attrs, cv, std::span<const TensorView>(ins3, bias ? 3 : 2), ctx, nullptr);
}

int32_t ref_requant_s8(int32_t acc, float req, int32_t zp)
{
    return backend::cpu::matmul_int8_requant<int8_t>(acc, req, zp);
}

int32_t ref_requant_u8(int32_t acc, float req, int32_t zp)
{
    return backend::cpu::matmul_int8_requant<uint8_t>(acc, req, zp);
}

float ref_requant_scale(float s_a, float s_b, float s_out)
{
    return backend::cpu::matmul_int8_requant_scale(s_a, s_b, s_out);
}

void ref_q4_1_quantize(const float* src, int64_t count, void* blocks)
{
    quantize_q4<float>(src, count, blocks);
}

void ref_q4_1_decode(const void* blocks, int64_t count, float* out)
{
    pack_q4<float>(blocks, count, out);
}

float ref_gelu(float x)
{
    Epilogue ep{};
    ep.type = EpilogueActivateType::Gelu;
    return apply_epilogue(ep, x);
}

uint16_t ref_f32_to_f16(float f)
{
    return half_to_bits(float_to_half(f));
}

float ref_f16_to_f32(uint16_t h)
{
    return half_to_float(half_from_bits(h));
}

}  // extern "C"
