#pragma once
/// @file quant_linear.hpp
/// @brief QuantizeLinear / DequantizeLinear on the HIP backend.
///
/// nnops' operators (include/nnops/ops/quant_linear.hpp:26-140,
/// src/ops/quant_linear.cpp): inputs x, scale (f32), zero point (s8/u8), one
/// output of x's shape.
///   QuantizeLinear    f32/f16 -> s8/u8:
///                     y = clamp(rint(fma(x, 1/scale, zero_point)), qmin, qmax),
///                     ties to even; NaN and |v| >= 2^31 give qmin.
///   DequantizeLinear  s8/u8 -> f32/f16: y = (x - zero_point) * scale, as one
///                     fma(x, scale, -zero_point*scale) over the whole
///                     16-element blocks of each row and the plain form over
///                     the row's last (row % 16) elements, like the x86 kernel.
/// Granularity follows the scale's size and `axis` (ONNX): one scale ->
/// per tensor; axis < 0 -> per token (one per innermost row); axis >= 0 -> per
/// channel along `axis`. The scale and zero-point tensors are device memory.

#include "nnops/core/op_base.hpp"

#include <cstdint>
#include <memory>

namespace nnops {

struct QuantLinearAttributes {
    int64_t axis = -1;
    /// QuantizeLinear: s8/u8. DequantizeLinear: f32/f16; any other value
    /// resolves to f32 at construction (nnops' rule).
    DataType output_dtype = DataType::s8;
};

class QuantizeLinear : public OpBase {
public:
    static std::unique_ptr<QuantizeLinear> create(const QuantLinearAttributes& attrs = {},
                                                  Backend backend = Backend::HIP);

    std::vector<TensorDesc> getOutputTensorDesc(std::span<const TensorDesc> inputs) const override;
    Status validate(std::span<const TensorDesc> inputs,
                    std::span<const TensorDesc> outputs) const override;
    using OpBase::compute;
    Status compute(std::span<TensorView> outputs, std::span<const TensorView> inputs,
                   const ComputeContext& ctx = {}, void* workspace = nullptr) override;
    Backend getBackend() const override { return backend_; }
    const QuantLinearAttributes& attributes() const noexcept { return attrs_; }

private:
    QuantizeLinear(const QuantLinearAttributes& attrs, Backend backend) : attrs_(attrs), backend_(backend) {}
    QuantLinearAttributes attrs_;
    Backend backend_;
};

class DequantizeLinear : public OpBase {
public:
    static std::unique_ptr<DequantizeLinear> create(const QuantLinearAttributes& attrs = {},
                                                    Backend backend = Backend::HIP);

    std::vector<TensorDesc> getOutputTensorDesc(std::span<const TensorDesc> inputs) const override;
    Status validate(std::span<const TensorDesc> inputs,
                    std::span<const TensorDesc> outputs) const override;
    using OpBase::compute;
    Status compute(std::span<TensorView> outputs, std::span<const TensorView> inputs,
                   const ComputeContext& ctx = {}, void* workspace = nullptr) override;
    Backend getBackend() const override { return backend_; }
    const QuantLinearAttributes& attributes() const noexcept { return attrs_; }

private:
    DequantizeLinear(const QuantLinearAttributes& attrs, Backend backend);
    QuantLinearAttributes attrs_;
    Backend backend_;
};

}  // namespace nnops
