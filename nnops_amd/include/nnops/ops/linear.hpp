#pragma once
/// @file linear.hpp
/// @brief Linear: output = epilogue(input x weight^T + bias) [+ residual].
///
/// nnops' Linear (include/nnops/ops/linear.hpp:41-142, src/ops/linear.cpp):
/// the weight is [N, K], the product is MatMul with transpose_b, the input is
/// [..., K] and the output [..., N]. For an integer pair the output follows
/// `output_dtype`: s32/s8/u8, or f32/f16 dequantized (bias in the output
/// dtype, any activation); a q4_1 weight with an f16/f32 input follows the
/// input dtype. add_to on an fp output folds into the sum before the clip when
/// residual_pre_activation is set or the epilogue is the identity, and is
/// added to the (destination-typed) activation otherwise
/// (src/backend/cpu/matmul/linear.cpp:276-301).
///
/// add_to on an s8/u8 destination (nnops rejects it, linear.cpp:224-226) is
/// defined here through the float epilogue: the old destination, dequantized
/// with the output's scale and zero point, joins the f32 sum after the
/// activation (or before it with residual_pre_activation), and the sum is
/// requantized.

#include "nnops/core/epilogue.hpp"
#include "nnops/core/op_base.hpp"

#include <limits>
#include <memory>

namespace nnops {

struct LinearAttributes {
    Epilogue epilogue{};
    bool add_to = false;
    bool residual_pre_activation = false;
    DataType output_dtype = DataType::f32;

    bool gated = false;  ///< fp-only in nnops; unsupported on the quantized routes
    EpilogueActivateType gate_activation = EpilogueActivateType::Silu;
    float gate_alpha = 1.0f;
    float gate_beta = 0.0f;
    float gate_limit = std::numeric_limits<float>::infinity();

    bool requant_round_even = false;
    bool float_epilogue = false;
};

class Linear : public OpBase {
public:
    static std::unique_ptr<Linear> create(const LinearAttributes& attrs, Backend backend = Backend::HIP);
    static std::unique_ptr<Linear> create(Backend backend = Backend::HIP)
    {
        return create(LinearAttributes{}, backend);
    }

    std::vector<TensorDesc> getOutputTensorDesc(std::span<const TensorDesc> inputs) const override;
    Status validate(std::span<const TensorDesc> inputs,
                    std::span<const TensorDesc> outputs) const override;
    size_t getWorkspaceSize(std::span<const TensorDesc> inputs,
                            std::span<const TensorDesc> outputs) const override;
    using OpBase::compute;
    Status compute(std::span<TensorView> outputs, std::span<const TensorView> inputs,
                   const ComputeContext& ctx = {}, void* workspace = nullptr) override;
    /// Query (empty outputs[0]: the packed descriptor is written back) or fill
    /// the prepacked weight (src/ops/matmul.cpp:96-141). An s8 weight packs
    /// into TensorLayout::PackedBHip; any other weight answers the query with
    /// an empty view (no packed form).
    void prepackWeights(std::span<const TensorView> inputs, std::span<TensorView> outputs,
                        const ComputeContext& ctx = {}) override;
    /// prepackWeights with its status (nnops asserts where this returns).
    Status prepack(std::span<const TensorView> inputs, std::span<TensorView> outputs,
                   const ComputeContext& ctx = {});
    Backend getBackend() const override { return backend_; }
    const LinearAttributes& attributes() const noexcept { return attrs_; }

private:
    Linear(const LinearAttributes& attrs, Backend backend) : attrs_(attrs), backend_(backend) {}
    LinearAttributes attrs_;
    Backend backend_;
};

}  // namespace nnops
