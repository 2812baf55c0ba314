// QuantizeLinear / DequantizeLinear for Backend::HIP: nnops' descriptor and
// dtype rules (src/ops/quant_linear.cpp:60-150), the granularity mapping of
// src/backend/cpu/quant_linear.cpp:92-118, lowered onto the C ABI entry points
// nnops_hip_quantize_linear / nnops_hip_dequantize_linear.
#include "nnops/ops/quant_linear.hpp"
#include "nnops_amd.h"

#include <hip/hip_runtime.h>

namespace nnops {
namespace {

bool rows_compact(const TensorDesc& d)
{
    return d.rank < 2 || d.row_stride_elems == 0 || d.row_stride_elems == d.cols();
}

/// The shared dtype rules: a float side, an s8/u8 side, an f32 scale and an
/// s8/u8 zero point; the kernels walk compact rows.
Status check_dtypes(std::span<const TensorDesc> inputs, std::span<const TensorDesc> outputs,
                    bool quantize)
{
    if (inputs.size() != 3 || outputs.size() != 1) {
        return Status::invalid_argument;
    }
    const DataType flt = quantize ? inputs[0].dtype : outputs[0].dtype;
    const DataType qnt = quantize ? outputs[0].dtype : inputs[0].dtype;
    if (flt != DataType::f32 && flt != DataType::f16) {
        return Status::unsupported;
    }
    if (qnt != DataType::s8 && qnt != DataType::u8) {
        return Status::invalid_argument;
    }
    if (inputs[1].dtype != DataType::f32) {
        return Status::invalid_argument;
    }
    if (inputs[2].dtype != DataType::s8 && inputs[2].dtype != DataType::u8) {
        return Status::invalid_argument;
    }
    if (!rows_compact(inputs[0]) || !rows_compact(outputs[0])) {
        return Status::unsupported;
    }
    return Status::ok;
}

int32_t kind_of(DataType dt)
{
    switch (dt) {
    case DataType::f32: return NNOPS_OUT_F32;
    case DataType::f16: return NNOPS_OUT_F16;
    case DataType::s8: return NNOPS_OUT_S8;
    case DataType::u8: return NNOPS_OUT_U8;
    default: return -1;
    }
}

Status from_code(int c)
{
    switch (c) {
    case NNOPS_OK: return Status::ok;
    case NNOPS_INVALID_ARGUMENT: return Status::invalid_argument;
    case NNOPS_UNSUPPORTED: return Status::unsupported;
    default: return Status::internal;
    }
}

/// Lower one call: x/y flat over numel elements as [total_rows, cols]; the
/// parameter of flat element i is (i / inner) % dim.
Status run(const QuantLinearAttributes& attrs, TensorView& y, std::span<const TensorView> inputs,
           const ComputeContext& ctx, bool quantize)
{
    const TensorView& x = inputs[0];
    const TensorView& scale = inputs[1];
    const TensorView& zp = inputs[2];
    if (x.rank() != y.rank() || x.numel() != y.numel()) {
        return Status::invalid_argument;
    }
    for (int64_t d = 0; d < x.rank(); ++d) {
        if (x.shape(d) != y.shape(d)) {
            return Status::invalid_argument;
        }
    }
    const int64_t numel = x.numel();
    if (numel == 0) {
        return Status::ok;
    }
    const int64_t rank = x.rank();
    const int64_t cols = rank > 0 ? x.shape(rank - 1) : 1;
    const int64_t nparams = scale.numel();
    if (zp.numel() != nparams) {
        return Status::invalid_argument;
    }
    int64_t inner = 1, dim = 1, segment = numel;
    if (nparams > 1) {
        if (attrs.axis < 0) {  // per token
            inner = cols;
            dim = numel / cols;
            segment = cols;
        } else {               // per channel
            if (attrs.axis >= rank) {
                return Status::invalid_argument;
            }
            dim = x.shape(attrs.axis);
            for (int64_t d = attrs.axis + 1; d < rank; ++d) {
                inner *= x.shape(d);
            }
            segment = inner;
        }
        if (nparams != dim) {
            return Status::invalid_argument;
        }
    } else if (nparams != 1) {
        return Status::invalid_argument;
    }
    NnopsQdqArgs a{};
    a.x = x.ptr<const void>();
    a.y = y.ptr<void>();
    a.rows = numel / cols;
    a.cols = cols;
    a.ld_x = cols;
    a.ld_y = cols;
    a.x_kind = kind_of(x.data_type());
    a.y_kind = kind_of(y.data_type());
    a.zp_kind = kind_of(zp.data_type());
    a.scale = scale.ptr<const float>();
    a.zero_point = zp.ptr<const void>();
    a.inner = inner;
    a.dim = dim;
    a.segment = segment;
    const int rc = quantize ? nnops_hip_quantize_linear(&a, ctx.hip_stream)
                            : nnops_hip_dequantize_linear(&a, ctx.hip_stream);
    return from_code(rc);
}

Status check_views(std::span<TensorView> outputs, std::span<const TensorView> inputs)
{
    if (inputs.size() != 3 || outputs.size() != 1) {
        return Status::invalid_argument;
    }
    for (const TensorView& v : inputs) {
        if (v.is_empty() && v.numel() != 0) {
            return Status::invalid_argument;
        }
    }
    if (outputs[0].is_empty() && outputs[0].numel() != 0) {
        return Status::invalid_argument;
    }
    return Status::ok;
}

std::vector<TensorDesc> same_shape(std::span<const TensorDesc> inputs, DataType dt)
{
    if (inputs.empty()) {
        return {};
    }
    TensorDesc d = inputs[0];
    d.dtype = dt;
    d.row_stride_elems = 0;
    return {d};
}

Status compute_common(const QuantLinearAttributes& attrs, Backend backend, std::span<TensorView> outputs,
                      std::span<const TensorView> inputs, const ComputeContext& ctx, bool quantize)
{
    if (Status s = check_views(outputs, inputs); !is_ok(s)) {
        return s;
    }
    if (backend != Backend::HIP) {
        return Status::unsupported;
    }
    const TensorDesc din[3] = {inputs[0].desc(), inputs[1].desc(), inputs[2].desc()};
    const TensorDesc dout = outputs[0].desc();
    if (Status s = check_dtypes(din, std::span<const TensorDesc>(&dout, 1), quantize); !is_ok(s)) {
        return s;
    }
    return run(attrs, outputs[0], inputs, ctx, quantize);
}

}  // namespace

std::unique_ptr<QuantizeLinear> QuantizeLinear::create(const QuantLinearAttributes& attrs, Backend backend)
{
    return std::unique_ptr<QuantizeLinear>(new QuantizeLinear(attrs, backend));
}

std::vector<TensorDesc> QuantizeLinear::getOutputTensorDesc(std::span<const TensorDesc> inputs) const
{
    return same_shape(inputs, attrs_.output_dtype);
}

Status QuantizeLinear::validate(std::span<const TensorDesc> inputs, std::span<const TensorDesc> outputs) const
{
    return check_dtypes(inputs, outputs, true);
}

Status QuantizeLinear::compute(std::span<TensorView> outputs, std::span<const TensorView> inputs,
                               const ComputeContext& ctx, void* workspace)
{
    (void)workspace;
    return compute_common(attrs_, backend_, outputs, inputs, ctx, true);
}

DequantizeLinear::DequantizeLinear(const QuantLinearAttributes& attrs, Backend backend)
    : attrs_(attrs), backend_(backend)
{
    // a dequantize output is always float: an integer request means f32
    if (attrs_.output_dtype != DataType::f32 && attrs_.output_dtype != DataType::f16) {
        attrs_.output_dtype = DataType::f32;
    }
}

std::unique_ptr<DequantizeLinear> DequantizeLinear::create(const QuantLinearAttributes& attrs, Backend backend)
{
    return std::unique_ptr<DequantizeLinear>(new DequantizeLinear(attrs, backend));
}

std::vector<TensorDesc> DequantizeLinear::getOutputTensorDesc(std::span<const TensorDesc> inputs) const
{
    return same_shape(inputs, attrs_.output_dtype);
}

Status DequantizeLinear::validate(std::span<const TensorDesc> inputs, std::span<const TensorDesc> outputs) const
{
    return check_dtypes(inputs, outputs, false);
}

Status DequantizeLinear::compute(std::span<TensorView> outputs, std::span<const TensorView> inputs,
                                 const ComputeContext& ctx, void* workspace)
{
    (void)workspace;
    return compute_common(attrs_, backend_, outputs, inputs, ctx, false);
}

}  // namespace nnops
