#pragma once
/// @file matmul.hpp
/// @brief MatMul: C = epilogue(A x B) — the quantized routes on the HIP backend.
///
/// The class, attributes and routing rules are nnops' (include/nnops/ops/
/// matmul.hpp:33-135, src/ops/matmul.cpp:40-152):
///   - an integer pair (s8|u8 A x s8 B, is_int8_matmul) takes its output dtype
///     from `output_dtype`: s32 is the raw MatMulInteger accumulate, s8/u8
///     requantize with the output view's QuantParams (or the epilogue's
///     Requantize table), half away from zero; f32/f16 dequantize
///     (v * s_a * s_b + bias, [residual], clip, activation);
///   - an fp A (f32/f16) with active per-tensor / per-token QuantParams
///     against an s8 B (is_fp_quant_matmul) is quantized to act_quant_dtype
///     with those parameters and dequantized back into A's dtype;
///   - an fp A (f16/f32) against a q4_1 B is the Q4_1 weight route; the output
///     dtype follows A, and an f32 destination for an f16 A is accepted too.
/// The optional third input is the [N] bias: int32 on integer destinations,
/// the output dtype on f32/f16 ones.
///
/// Extensions (off by default, so nnops semantics are untouched):
///   requant_round_even  round half to even in the requant instead;
///   float_epilogue      produce an s8/u8 destination through the f32
///                       epilogue (dequant -> clip -> activation, GELU
///                       included -> residual -> requant) instead of the
///                       integer pass, which honours only Relu.

#include "nnops/core/epilogue.hpp"
#include "nnops/core/op_base.hpp"

#include <memory>

namespace nnops {

struct MatMulAttributes {
    bool transpose_a = false;
    bool transpose_b = false;
    float alpha = 1.0f;   ///< ignored by the integer routes (as in nnops)
    float beta = 0.0f;    ///< ignored by the integer routes (as in nnops)
    bool residual_pre_activation = false;
    DataType output_dtype = DataType::s32;
    DataType act_quant_dtype = DataType::s8;
    Epilogue epilogue{};

    bool requant_round_even = false;
    bool float_epilogue = false;
};

inline constexpr bool is_int8_matmul(DataType a, DataType b) noexcept
{
    return (a == DataType::s8 || a == DataType::u8) && b == DataType::s8;
}

inline constexpr bool is_q4_1_matmul(DataType a, DataType b) noexcept
{
    return (a == DataType::f32 || a == DataType::f16) && b == DataType::q4_1;
}

class MatMul : public OpBase {
public:
    static std::unique_ptr<MatMul> create(const MatMulAttributes& attrs = {},
                                          Backend backend = Backend::HIP);

    std::vector<TensorDesc> getOutputTensorDesc(std::span<const TensorDesc> inputs) const override;
    Status validate(std::span<const TensorDesc> inputs,
                    std::span<const TensorDesc> outputs) const override;
    size_t getWorkspaceSize(std::span<const TensorDesc> inputs,
                            std::span<const TensorDesc> outputs) const override;
    using OpBase::compute;
    Status compute(std::span<TensorView> outputs, std::span<const TensorView> inputs,
                   const ComputeContext& ctx = {}, void* workspace = nullptr) override;
    /// Query (empty outputs[0]: the packed descriptor is written back) or fill
    /// the prepacked weight (src/ops/matmul.cpp:96-141). An s8 weight, and a
    /// q4_1 weight with blocks along N (transpose_b false), pack into
    /// TensorLayout::PackedBHip; any other weight answers the query with an
    /// empty view (no packed form).
    void prepackWeights(std::span<const TensorView> inputs, std::span<TensorView> outputs,
                        const ComputeContext& ctx = {}) override;
    /// prepackWeights with its status (nnops asserts where this returns).
    Status prepack(std::span<const TensorView> inputs, std::span<TensorView> outputs,
                   const ComputeContext& ctx = {});
    Backend getBackend() const override { return backend_; }
    const MatMulAttributes& attributes() const noexcept { return attrs_; }

private:
    MatMul(const MatMulAttributes& attrs, Backend backend) : attrs_(attrs), backend_(backend) {}
    MatMulAttributes attrs_;
    Backend backend_;
};

}  // namespace nnops
