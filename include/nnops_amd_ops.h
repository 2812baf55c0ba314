/* nnops_amd_ops.h -- C ABI over the MatMul / Linear / QuantizeLinear /
 * DequantizeLinear front end.
 *
 * For callers that cannot bind C++ (ctypes, cgo, JNI, N-API): each call maps
 * one-to-one onto the C++ operator contract of nnops
 * (include/nnops/core/op_base.hpp:30-115, include/nnops/ops/matmul.hpp:88-135,
 * include/nnops/ops/linear.hpp:89-142): create -> output_desc -> validate ->
 * workspace_size -> compute, over caller-owned device buffers described by
 * NnopsTensor (a flattened TensorView: shape, dtype, data, pitch, QuantParams).
 * Status values are nnops::Status's (see nnops_amd.h). No call allocates
 * device memory; compute enqueues on `hip_stream` and returns.
 */
#ifndef NNOPS_AMD_OPS_H
#define NNOPS_AMD_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* nnops::DataType values (include/nnops/core/data_type.hpp:23-36) */
enum {
    NNOPS_F32 = 0, NNOPS_F16 = 1, NNOPS_BF16 = 2, NNOPS_S8 = 3, NNOPS_U8 = 4,
    NNOPS_S32 = 5, NNOPS_S64 = 6, NNOPS_Q4_1 = 11,
};

/* nnops::Backend values; NNOPS_BACKEND_HIP is the one with kernels here */
enum { NNOPS_BACKEND_CPU = 0, NNOPS_BACKEND_CUDA = 1, NNOPS_BACKEND_HIP = 4 };

typedef struct NnopsTensor {
    int64_t rank;
    int64_t dims[8];
    int32_t dtype;          /* NNOPS_F32 ... */
    void* data;             /* device pointer; NULL = descriptor only */
    int64_t pitch;          /* bytes between rows; 0 = dense */
    /* QuantParams (include/nnops/core/quant_params.hpp:36-61) */
    int32_t granularity;    /* 0 per-tensor, 1 per-token, 2 per-channel */
    float scale;
    int32_t zero_point;
    const float* scale_data;        /* host or device */
    const int32_t* zero_point_data; /* host or device */
    int64_t num_scales;
    int32_t layout;         /* nnops::TensorLayout value; 0 = Dense (12). 18 = PackedBHip,
                               the prepacked weight nnops_op_prepack_weights describes */
} NnopsTensor;

/* nnops::Epilogue (include/nnops/core/epilogue.hpp:73-92) */
typedef struct NnopsEpilogue {
    int32_t type;           /* EpilogueActivateType value */
    float alpha, beta, min_clip, max_clip;
    int32_t quant;          /* EpilogueQuantType value */
    const float* quant_scales;
    const int32_t* quant_zero_points;
    int64_t quant_param_count;
} NnopsEpilogue;

typedef struct NnopsMatMulAttrs {
    int32_t transpose_a, transpose_b;
    float alpha, beta;
    int32_t residual_pre_activation;
    int32_t output_dtype;
    NnopsEpilogue epilogue;
    int32_t requant_round_even;  /* extension */
    int32_t float_epilogue;      /* extension */
    /* storage of the fp-activation quantization (NNOPS_S8 / NNOPS_U8),
       MatMulAttributes::act_quant_dtype (include/nnops/ops/matmul.hpp:62-64) */
    int32_t act_quant_dtype;
} NnopsMatMulAttrs;

typedef struct NnopsLinearAttrs {
    NnopsEpilogue epilogue;
    int32_t add_to, residual_pre_activation;
    int32_t output_dtype;
    int32_t gated;
    int32_t requant_round_even;  /* extension */
    int32_t float_epilogue;      /* extension */
    /* the gated form (LinearAttributes::gate_*, include/nnops/ops/linear.hpp:
       71-88): gate activation (NNOPS_ACT_SILU default, GELU, RELU, SIGMOID,
       TANH, NONE), alpha (Silu), beta, limit (+inf: no clamp) */
    int32_t gate_activation;
    float gate_alpha, gate_beta, gate_limit;
} NnopsLinearAttrs;

/* nnops::QuantLinearAttributes (include/nnops/ops/quant_linear.hpp:26-35) */
typedef struct NnopsQuantLinearAttrs {
    int64_t axis;           /* -1 per token; >= 0 per channel (one scale: per tensor) */
    int32_t output_dtype;   /* quantize: NNOPS_S8 / NNOPS_U8; dequantize: NNOPS_F32 / NNOPS_F16 */
} NnopsQuantLinearAttrs;

typedef struct NnopsOp NnopsOp;

/* Attribute defaults matching the C++ structs (epilogue clip +-inf etc.). */
void nnops_matmul_attrs_init(NnopsMatMulAttrs* attrs);
void nnops_linear_attrs_init(NnopsLinearAttrs* attrs);

NnopsOp* nnops_matmul_create(const NnopsMatMulAttrs* attrs, int32_t backend);
NnopsOp* nnops_linear_create(const NnopsLinearAttrs* attrs, int32_t backend);
/* QuantizeLinear / DequantizeLinear (include/nnops/ops/quant_linear.hpp:47-140):
 * inputs x, scale (f32, device), zero point (s8/u8, device, scale's size). */
void nnops_quant_linear_attrs_init(NnopsQuantLinearAttrs* attrs);
NnopsOp* nnops_quantize_linear_create(const NnopsQuantLinearAttrs* attrs, int32_t backend);
NnopsOp* nnops_dequantize_linear_create(const NnopsQuantLinearAttrs* attrs, int32_t backend);
void nnops_op_destroy(NnopsOp* op);

/* OpBase::prepackWeights (include/nnops/core/op_base.hpp:72-78) for MatMul /
 * Linear: with outputs[0].data == NULL it is the query and writes the packed
 * descriptor (dims, dtype, pitch, layout = 18; rank 0 = no packed form) into
 * outputs[0]; with outputs[0] describing a device buffer of that size (256-byte
 * aligned) it fills it on `hip_stream`. inputs[0] is the raw weight. Returns a
 * Status. The packed weight then goes to compute() as the B / weight input. */
int nnops_op_prepack_weights(NnopsOp* op, const NnopsTensor* inputs, int32_t n_inputs, NnopsTensor* outputs,
                             int32_t n_outputs, void* hip_stream);

/* Fills out_desc (dims, rank, dtype; data NULL). Returns 0 on success. */
int nnops_op_output_desc(const NnopsOp* op, const NnopsTensor* inputs, int32_t n_inputs,
                         NnopsTensor* out_desc);
int nnops_op_validate(const NnopsOp* op, const NnopsTensor* inputs, int32_t n_inputs,
                      const NnopsTensor* outputs, int32_t n_outputs);
size_t nnops_op_workspace_size(const NnopsOp* op, const NnopsTensor* inputs, int32_t n_inputs,
                               const NnopsTensor* outputs, int32_t n_outputs);
int nnops_op_compute(NnopsOp* op, const NnopsTensor* outputs, int32_t n_outputs,
                     const NnopsTensor* inputs, int32_t n_inputs, void* hip_stream,
                     void* workspace);

#ifdef __cplusplus
}
#endif

#endif /* NNOPS_AMD_OPS_H */
