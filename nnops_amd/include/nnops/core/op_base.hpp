#pragma once
/// @file op_base.hpp
/// @brief OpBase — the operator contract (include/nnops/core/op_base.hpp:30-115
/// in nnops): getOutputTensorDesc -> validate -> getWorkspaceSize -> compute
/// over caller-owned views and a caller-owned workspace; compute never
/// allocates and a rejected call writes nothing.

#include "nnops/core/backend.hpp"
#include "nnops/core/compute_context.hpp"
#include "nnops/core/status.hpp"
#include "nnops/core/tensor_view.hpp"

#include <cstddef>
#include <span>
#include <vector>

namespace nnops {

class OpBase {
public:
    virtual ~OpBase() = default;

    virtual std::vector<TensorDesc> getOutputTensorDesc(std::span<const TensorDesc> inputs) const = 0;

    virtual size_t getWorkspaceSize(std::span<const TensorDesc> inputs,
                                    std::span<const TensorDesc> outputs) const
    {
        (void)inputs;
        (void)outputs;
        return 0;
    }

    virtual Status validate(std::span<const TensorDesc> inputs,
                            std::span<const TensorDesc> outputs) const
    {
        (void)inputs;
        (void)outputs;
        return Status::ok;
    }

    virtual Status compute(std::span<TensorView> outputs, std::span<const TensorView> inputs,
                           const ComputeContext& ctx = {}, void* workspace = nullptr) = 0;

    /// Single-output convenience overload (op_base.hpp:63-70 in nnops).
    Status compute(TensorView& output, std::span<const TensorView> inputs,
                   const ComputeContext& ctx = {}, void* workspace = nullptr)
    {
        TensorView outs[] = {output};
        return compute(std::span<TensorView>(outs), inputs, ctx, workspace);
    }

    /// Two-step weight prepack: an empty outputs[0] is the query. Weights with
    /// no packed form answer the query with an empty view.
    virtual void prepackWeights(std::span<const TensorView> inputs, std::span<TensorView> outputs,
                                const ComputeContext& ctx = {})
    {
        (void)inputs;
        (void)outputs;
        (void)ctx;
    }

    virtual Backend getBackend() const = 0;
};

}  // namespace nnops
