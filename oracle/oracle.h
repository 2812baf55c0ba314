/* CPU oracle for the quantized-matmul path (test infrastructure only).
 *
 * This is the checker the HIP path is compared against. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it; the product
 * library never links or calls it.
 *
 * Every function restates the reference algorithm it names (paths relative to
 * the nnops source tree) in plain C99 with no vector intrinsics, compiled with
 * -ffp-contract=off so each float operation rounds on its own, as in the
 * reference's scalar code.
 *
 * Pinning (what checks each function beyond its own formula):
 *   orc_gemm_i8 int32/s8/u8 outputs  known answers of tests/test_matmul_int8.cpp,
 *                                    brute-force int64 matmul, golden vectors
 *                                    from the compiled reference oracle.
 *   orc_gemm_i8 f32/f16 (dq) output  the compiled reference matmul_dq_ref (when
 *                                    built) on the same int8 operands, bit for
 *                                    bit, and the known answers of
 *                                    tests/test_matmul_dq.cpp:185-247.
 *   orc_gemm_i8 float epilogue       s8 add_to / gelu on an integer destination:
 *                                    no reference route exists, so the composite
 *                                    is PARITY UNPINNED; its pieces are pinned
 *                                    (int accumulate, dq scale, GELU values vs
 *                                    the reference's std::tanh GELU within 2 ulp
 *                                    of the output scale).
 *   orc_f32_to_f16/orc_f16_to_f32    exhaustive vs numpy float16 (IEEE RNE).
 *   orc_q4_1_*                       llama.cpp known answers restated in
 *                                    tests/test_q4_1.cpp, golden bytes from the
 *                                    compiled reference quantize_q4.
 *   orc_gemm_q4_1                    float64 brute force from decoded weights.
 *   orc_quantize/dequantize_linear   known answers of tests/test_quant_linear.cpp
 *                                    (ties to even, clamps, per-channel and
 *                                    per-token indexing, u8 zero points), exact
 *                                    rational checks (power-of-two scales), and
 *                                    the round trip q -> x -> q.
 */
#ifndef NNOPS_ORACLE_H
#define NNOPS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_OUT_S32 = 0, ORC_OUT_S8 = 1, ORC_OUT_U8 = 2, ORC_OUT_F32 = 3, ORC_OUT_F16 = 4 };
/* EpilogueActivateType values (include/nnops/core/epilogue.hpp:25-36) */
enum {
    ORC_ACT_NONE = 0, ORC_ACT_RELU = 1, ORC_ACT_GELU = 2, ORC_ACT_SIGMOID = 3, ORC_ACT_TANH = 4,
    ORC_ACT_LEAKY_RELU = 5, ORC_ACT_SILU = 6, ORC_ACT_HARDSWISH = 7, ORC_ACT_ELU = 8, ORC_ACT_RELU6 = 9
};

typedef struct {
    const void* a;        /* s8 or u8, [M,K] (or [K,M] with trans_a) */
    const int8_t* b;      /* s8, [K,N] (or [N,K] with trans_b) */
    const void* bias;     /* [N]: int32 for integer outputs, f32 / f16 bits for ORC_OUT_F32 / F16; may be NULL */
    void* c;              /* destination (f16 as its bits); read first when add_to */
    int64_t m, n, k;
    int64_t lda, ldb, ldc; /* row strides in elements */
    int32_t trans_a, trans_b, a_u8;
    /* quantization (arrays override scalars when non-NULL) */
    const float* s_a; float s_a_scalar; const int32_t* zp_a; int32_t zp_a_scalar;
    const float* s_b; float s_b_scalar; const int32_t* zp_b; int32_t zp_b_scalar;
    const float* s_out_rows; const int32_t* zp_out_rows; float s_out; int32_t zp_out;
    int32_t out_kind;     /* ORC_OUT_* */
    int32_t act;          /* ORC_ACT_*; integer route honours only RELU */
    int32_t round_even;   /* 0: half away from zero (nnops), 1: half to even */
    /* float epilogue on an integer destination (extension, see header) */
    int32_t float_ep;
    float min_clip, max_clip;
    int32_t add_to, residual_pre;
    /* rows [m_begin, m_end) are computed; m_end <= 0 means all rows */
    int64_t m_begin, m_end;
    float act_alpha, act_beta;  /* LeakyRelu / Elu alpha, HardSwish beta */
} orc_gemm_i8_t;

void orc_gemm_i8(const orc_gemm_i8_t* p);

/* Scalar requant of one compensated accumulate (simd_epilogue.hpp:137-147). */
int32_t orc_requant(int32_t acc, float req, int32_t zp, int32_t u8, int32_t round_even);
float orc_requant_scale(float s_a, float s_b, float s_out);

float orc_tanhf(float x);
int64_t orc_markstein_mismatches(float b, uint32_t lo, uint32_t hi, uint32_t step, int32_t corrected);
float orc_gelu_tanh(float x);

uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);

void orc_q4_1_decode(const void* blocks, int64_t count, float* out);
void orc_q4_1_quantize(const float* src, int64_t count, void* blocks);

typedef struct {
    const void* a;        /* f16 (a_f16) or f32, [M,K] */
    const uint8_t* b;     /* Q4_1 blocks: trans_b -> [N][ceil(K/32)], else [K][ceil(N/32)] */
    void* c;              /* f32 or f16 (c_f16), [M,N] */
    int64_t m, n, k;
    int64_t lda, ldc;     /* elements */
    int64_t ldb_bytes;    /* bytes between B rows */
    int32_t trans_b, a_f16, c_f16;
    int32_t w_round_f16;  /* round each decoded weight to f16 (nnops f16-A semantics) */
    int32_t acc_f64;      /* accumulate in double (1) or float (0) */
    int64_t m_begin, m_end;
} orc_gemm_q4_1_t;

void orc_gemm_q4_1(const orc_gemm_q4_1_t* p);

/* The fp output pass after a Q4_1 GEMM (f32 results src [rows][ld_src]):
 * bias, residual and epilogue, or Linear's gated combine. See orc_fp_out_pass
 * in oracle.c for the references it follows. */
typedef struct {
    const float* src;
    int64_t ld_src;
    void* out;            /* f32 or f16 (out_f16) [rows][ld_out] */
    int64_t ld_out, rows, n;
    int32_t out_f16;
    const void* bias;     /* out's type, [n] or gated [2n], or NULL */
    int32_t act;
    float act_alpha, act_beta, min_clip, max_clip;
    int32_t add_to, residual_pre, gated, gate_act;
    float gate_alpha, gate_beta, gate_limit;
    int32_t matmul_order;  /* MatMul's alpha P + T(beta old + bias) order */
    float alpha, beta;
} orc_fp_out_t;

void orc_fp_out_pass(const orc_fp_out_t* p);

/* QuantizeLinear / DequantizeLinear over `count` flat elements; element i
 * uses parameter (i / inner) % dim; `segment` is the reference kernel's row
 * length (numel per tensor, cols per token, inner per channel). */
void orc_quantize_linear(const void* x, int32_t x_f16, void* y, int32_t y_u8, int64_t count,
                         const float* scale, const int32_t* zero_point, int64_t inner, int64_t dim);
void orc_dequantize_linear(const void* x, int32_t x_u8, void* y, int32_t y_f16, int64_t count,
                           const float* scale, const int32_t* zero_point, int64_t inner, int64_t dim,
                           int64_t segment);

/* xorshift128+ stream of the reference test harness (random_tensor.hpp:18-57) */
void orc_xs128_u64(uint64_t seed, int64_t count, uint64_t* out);

#ifdef __cplusplus
}
#endif

#endif
