// C facade over the MatMul / Linear classes (include/nnops_amd_ops.h): turns
// NnopsTensor records into TensorDesc / TensorView and forwards each call.
#include "nnops/ops/linear.hpp"
#include "nnops/ops/matmul.hpp"
#include "nnops/ops/quant_linear.hpp"
#include "nnops_amd_ops.h"

#include <limits>
#include <memory>

using namespace nnops;

struct NnopsOp {
    std::unique_ptr<OpBase> op;
};

namespace {

TensorView to_view(const NnopsTensor& t)
{
    QuantParams qp;
    qp.granularity = static_cast<QuantGranularity>(t.granularity);
    qp.scale = t.scale;
    qp.zero_point = t.zero_point;
    qp.scale_data = t.scale_data;
    qp.zero_point_data = t.zero_point_data;
    qp.num_scales = t.num_scales;
    const int64_t rank = t.rank < 0 ? 0 : (t.rank > 8 ? 8 : t.rank);
    std::span<const int64_t> shape(t.dims, static_cast<size_t>(rank));
    const DataType dt = static_cast<DataType>(t.dtype);
    const TensorLayout lay = t.layout == 0 ? TensorLayout::Dense : static_cast<TensorLayout>(t.layout);
    if (t.pitch > 0) {
        return TensorView(shape, dt, t.data, t.pitch, lay, qp);
    }
    return TensorView(shape, dt, t.data, lay, qp);
}

Epilogue to_epilogue(const NnopsEpilogue& e)
{
    Epilogue ep;
    ep.type = static_cast<EpilogueActivateType>(e.type);
    ep.alpha = e.alpha;
    ep.beta = e.beta;
    ep.min_clip = e.min_clip;
    ep.max_clip = e.max_clip;
    ep.quant = static_cast<EpilogueQuantType>(e.quant);
    ep.quant_scales = e.quant_scales;
    ep.quant_zero_points = e.quant_zero_points;
    ep.quant_param_count = e.quant_param_count;
    return ep;
}

void init_epilogue(NnopsEpilogue& e)
{
    e.type = 0;
    e.alpha = 0.0f;
    e.beta = 1.0f;
    e.min_clip = -std::numeric_limits<float>::infinity();
    e.max_clip = std::numeric_limits<float>::infinity();
    e.quant = 0;
    e.quant_scales = nullptr;
    e.quant_zero_points = nullptr;
    e.quant_param_count = 0;
}

QuantLinearAttributes to_qlinear(const NnopsQuantLinearAttrs* a)
{
    QuantLinearAttributes attrs;
    if (a != nullptr) {
        attrs.axis = a->axis;
        attrs.output_dtype = static_cast<DataType>(a->output_dtype);
    }
    return attrs;
}

std::vector<TensorDesc> descs(const NnopsTensor* t, int32_t n)
{
    std::vector<TensorDesc> d;
    for (int32_t i = 0; i < n; ++i) {
        d.push_back(to_view(t[i]).desc());
    }
    return d;
}

}  // namespace

extern "C" {

void nnops_matmul_attrs_init(NnopsMatMulAttrs* a)
{
    if (a == nullptr) {
        return;
    }
    *a = NnopsMatMulAttrs{};
    a->alpha = 1.0f;
    a->beta = 0.0f;
    a->output_dtype = static_cast<int32_t>(DataType::s32);
    a->act_quant_dtype = static_cast<int32_t>(DataType::s8);
    init_epilogue(a->epilogue);
}

void nnops_linear_attrs_init(NnopsLinearAttrs* a)
{
    if (a == nullptr) {
        return;
    }
    *a = NnopsLinearAttrs{};
    a->output_dtype = static_cast<int32_t>(DataType::f32);
    init_epilogue(a->epilogue);
    const LinearAttributes d;
    a->gate_activation = static_cast<int32_t>(d.gate_activation);
    a->gate_alpha = d.gate_alpha;
    a->gate_beta = d.gate_beta;
    a->gate_limit = d.gate_limit;
}

NnopsOp* nnops_matmul_create(const NnopsMatMulAttrs* a, int32_t backend)
{
    MatMulAttributes attrs;
    if (a != nullptr) {
        attrs.transpose_a = a->transpose_a != 0;
        attrs.transpose_b = a->transpose_b != 0;
        attrs.alpha = a->alpha;
        attrs.beta = a->beta;
        attrs.residual_pre_activation = a->residual_pre_activation != 0;
        attrs.output_dtype = static_cast<DataType>(a->output_dtype);
        attrs.epilogue = to_epilogue(a->epilogue);
        attrs.requant_round_even = a->requant_round_even != 0;
        attrs.float_epilogue = a->float_epilogue != 0;
        attrs.act_quant_dtype = static_cast<DataType>(a->act_quant_dtype);
    }
    auto* h = new NnopsOp;
    h->op = MatMul::create(attrs, static_cast<Backend>(backend));
    return h;
}

NnopsOp* nnops_linear_create(const NnopsLinearAttrs* a, int32_t backend)
{
    LinearAttributes attrs;
    if (a != nullptr) {
        attrs.epilogue = to_epilogue(a->epilogue);
        attrs.add_to = a->add_to != 0;
        attrs.residual_pre_activation = a->residual_pre_activation != 0;
        attrs.output_dtype = static_cast<DataType>(a->output_dtype);
        attrs.gated = a->gated != 0;
        attrs.requant_round_even = a->requant_round_even != 0;
        attrs.float_epilogue = a->float_epilogue != 0;
        attrs.gate_activation = static_cast<EpilogueActivateType>(a->gate_activation);
        attrs.gate_alpha = a->gate_alpha;
        attrs.gate_beta = a->gate_beta;
        attrs.gate_limit = a->gate_limit;
    }
    auto* h = new NnopsOp;
    h->op = Linear::create(attrs, static_cast<Backend>(backend));
    return h;
}

void nnops_quant_linear_attrs_init(NnopsQuantLinearAttrs* a)
{
    if (a == nullptr) {
        return;
    }
    a->axis = -1;
    a->output_dtype = static_cast<int32_t>(DataType::s8);
}

NnopsOp* nnops_quantize_linear_create(const NnopsQuantLinearAttrs* a, int32_t backend)
{
    auto* h = new NnopsOp;
    h->op = QuantizeLinear::create(to_qlinear(a), static_cast<Backend>(backend));
    return h;
}

NnopsOp* nnops_dequantize_linear_create(const NnopsQuantLinearAttrs* a, int32_t backend)
{
    QuantLinearAttributes attrs = to_qlinear(a);
    if (a == nullptr) {
        attrs.output_dtype = DataType::f32;
    }
    auto* h = new NnopsOp;
    h->op = DequantizeLinear::create(attrs, static_cast<Backend>(backend));
    return h;
}

void nnops_op_destroy(NnopsOp* op)
{
    delete op;
}

int nnops_op_output_desc(const NnopsOp* op, const NnopsTensor* inputs, int32_t n_inputs,
                         NnopsTensor* out)
{
    if (op == nullptr || inputs == nullptr || out == nullptr || n_inputs < 2) {
        return static_cast<int>(Status::invalid_argument);
    }
    const std::vector<TensorDesc> in = descs(inputs, n_inputs);
    const std::vector<TensorDesc> o = op->op->getOutputTensorDesc(in);
    if (o.empty()) {
        return static_cast<int>(Status::invalid_argument);
    }
    *out = NnopsTensor{};
    out->rank = o[0].rank;
    for (int64_t i = 0; i < o[0].rank; ++i) {
        out->dims[i] = o[0].dims[static_cast<size_t>(i)];
    }
    out->dtype = static_cast<int32_t>(o[0].dtype);
    out->scale = 1.0f;
    return 0;
}

int nnops_op_prepack_weights(NnopsOp* op, const NnopsTensor* inputs, int32_t n_inputs, NnopsTensor* outputs,
                             int32_t n_outputs, void* hip_stream)
{
    if (op == nullptr || inputs == nullptr || outputs == nullptr || n_inputs < 1 || n_outputs < 1) {
        return static_cast<int>(Status::invalid_argument);
    }
    const TensorView in = to_view(inputs[0]);
    TensorView out[1] = {outputs[0].data != nullptr ? to_view(outputs[0]) : TensorView{}};
    ComputeContext ctx;
    ctx.hip_stream = hip_stream;
    Status st = Status::unsupported;
    if (auto* mm = dynamic_cast<MatMul*>(op->op.get())) {
        st = mm->prepack(std::span<const TensorView>(&in, 1), std::span<TensorView>(out, 1), ctx);
    } else if (auto* ln = dynamic_cast<Linear*>(op->op.get())) {
        st = ln->prepack(std::span<const TensorView>(&in, 1), std::span<TensorView>(out, 1), ctx);
    } else {
        // no packed form: the query answers empty
        st = outputs[0].data == nullptr ? Status::ok : Status::unsupported;
    }
    if (is_ok(st) && outputs[0].data == nullptr) {
        NnopsTensor d{};
        d.rank = out[0].rank();
        for (int64_t i = 0; i < d.rank; ++i) {
            d.dims[i] = out[0].shape(i);
        }
        d.dtype = static_cast<int32_t>(out[0].data_type());
        d.pitch = out[0].pitch();
        d.layout = d.rank > 0 ? static_cast<int32_t>(out[0].layout()) : 0;
        const QuantParams& qp = out[0].quant_params();
        d.granularity = static_cast<int32_t>(qp.granularity);
        d.scale = d.rank > 0 ? qp.scale : 1.0f;
        d.zero_point = qp.zero_point;
        d.scale_data = qp.scale_data;
        d.zero_point_data = qp.zero_point_data;
        d.num_scales = qp.num_scales;
        outputs[0] = d;
    }
    return static_cast<int>(st);
}

int nnops_op_validate(const NnopsOp* op, const NnopsTensor* inputs, int32_t n_inputs,
                      const NnopsTensor* outputs, int32_t n_outputs)
{
    if (op == nullptr || n_inputs < 0 || n_outputs < 0) {
        return static_cast<int>(Status::invalid_argument);
    }
    return static_cast<int>(op->op->validate(descs(inputs, n_inputs), descs(outputs, n_outputs)));
}

size_t nnops_op_workspace_size(const NnopsOp* op, const NnopsTensor* inputs, int32_t n_inputs,
                               const NnopsTensor* outputs, int32_t n_outputs)
{
    if (op == nullptr || n_inputs < 0 || n_outputs < 0) {
        return 0;
    }
    return op->op->getWorkspaceSize(descs(inputs, n_inputs), descs(outputs, n_outputs));
}

int nnops_op_compute(NnopsOp* op, const NnopsTensor* outputs, int32_t n_outputs,
                     const NnopsTensor* inputs, int32_t n_inputs, void* hip_stream, void* workspace)
{
    if (op == nullptr || n_inputs < 0 || n_outputs < 0 || n_inputs > 3 || n_outputs > 1) {
        return static_cast<int>(Status::invalid_argument);
    }
    TensorView in[3], out[1];
    for (int32_t i = 0; i < n_inputs; ++i) {
        in[i] = to_view(inputs[i]);
    }
    for (int32_t i = 0; i < n_outputs; ++i) {
        out[i] = to_view(outputs[i]);
    }
    ComputeContext ctx;
    ctx.hip_stream = hip_stream;
    return static_cast<int>(op->op->compute(std::span<TensorView>(out, static_cast<size_t>(n_outputs)),
                                            std::span<const TensorView>(in, static_cast<size_t>(n_inputs)),
                                            ctx, workspace));
}

}  // extern "C"
