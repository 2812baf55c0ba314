/* nnops_amd.h -- C ABI of the MI355X (gfx950) quantized-matmul path.
 *
 * This is the drop-in boundary below nnops' operator front end. In nnops the
 * CPU and CUDA backends are bound to `MatMul` / `Linear` through one kernel
 * function pointer per op, `Status fn(attrs, TensorView& out, span<const
 * TensorView> in, const ComputeContext&, void* workspace)`
 * (src/ops/dispatch.hpp:42-43, 62-96); the CUDA side of the integer route
 * flattens the views into a POD parameter block and launches on
 * `ctx.cuda_stream` (src/backend/cuda/matmul/matmul.cu:34-98,
 * src/backend/cuda/matmul/matmul_i8_common.cuh). The entry points below are
 * that launch boundary for a `Backend::HIP`: plain device pointers, element
 * strides taken from `TensorView::row_stride_elems()`, scalars, a
 * caller-provided device workspace and an opaque `hipStream_t`.
 *
 * Contract (all entry points):
 *   - every pointer in an args block is a DEVICE pointer (the C++ front end
 *     stages host QuantParams tables into the workspace);
 *   - nothing is allocated and nothing synchronises the host: work is enqueued
 *     on `stream` and the call returns;
 *   - `workspace` must hold at least the matching *_workspace_size() bytes
 *     (NNOPS_NOT_INITIALIZED otherwise) and must not be shared by calls that
 *     may run concurrently; its contents on entry are irrelevant;
 *   - a rejected call returns a non-zero status and enqueues nothing.
 */
#ifndef NNOPS_AMD_H
#define NNOPS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: nnops::Status values (include/nnops/core/status.hpp:19-33). */
enum {
    NNOPS_OK = 0,
    NNOPS_INVALID_ARGUMENT = 1,
    NNOPS_UNSUPPORTED = 2,
    NNOPS_NOT_INITIALIZED = 3,
    NNOPS_OUT_OF_MEMORY = 4,
    NNOPS_INTERNAL = 5,
};

/* Destination element types (nnops' s32/s8/u8 integer destinations,
 * MatMulAttributes::output_dtype, include/nnops/ops/matmul.hpp:53-60; f32/f16
 * for the Q4_1 route and the int8 route's dequantizing destinations). */
enum {
    NNOPS_OUT_S32 = 0,
    NNOPS_OUT_S8 = 1,
    NNOPS_OUT_U8 = 2,
    NNOPS_OUT_F32 = 3,
    NNOPS_OUT_F16 = 4,
};

/* Activations the output pass applies: EpilogueActivateType's values
 * (include/nnops/core/epilogue.hpp:25-36). The requantizing integer pass of
 * nnops honours only Relu (matmul_tile_impl.h:411); the float epilogue of an
 * s8/u8 destination takes None/Relu/Gelu; the dequantizing f32/f16
 * destinations take all of them. */
enum {
    NNOPS_ACT_NONE = 0,
    NNOPS_ACT_RELU = 1,
    NNOPS_ACT_GELU = 2,
    NNOPS_ACT_SIGMOID = 3,
    NNOPS_ACT_TANH = 4,
    NNOPS_ACT_LEAKY_RELU = 5,
    NNOPS_ACT_SILU = 6,
    NNOPS_ACT_HARDSWISH = 7,
    NNOPS_ACT_ELU = 8,
    NNOPS_ACT_RELU6 = 9,
};

/* Integer GEMM  C[M,N] = epilogue(A[M,K] x B[K,N]).
 * Replaces the integer route of nnops' matmul_cuda / linear_cuda
 * (src/backend/cuda/matmul/matmul.cu:34-98, GemmI8Params) and of matmul_cpu's
 * I8Route (src/backend/cpu/matmul/matmul_i8.cpp:55-159).
 *
 * A is s8 or u8 (a_u8), [M,K] row-major with row stride lda, or [K,M] with
 * trans_a. B is s8, [K,N] (ldb) or [N,K] with trans_b (Linear's weight).
 * Quantization tables override their scalars when non-null: s_a/zp_a per row
 * of A (PerToken), s_b/zp_b per output column (PerChannel), s_out_rows/
 * zp_out_rows per output row (Epilogue Requantize table).
 *
 * Output pass, per element, nnops order (simd_epilogue.hpp:341-467):
 *   v = sum (a - zp_a)(b - zp_b) + bias[n];  Relu;  for s8/u8:
 *   q = sat(round(clamp(float(v) * ((s_a / s_out) * s_b), lo - zp, hi - zp)) + zp)
 * with round = half away from zero (round_even = 0, nnops) or half to even.
 *
 * float_ep (extension, no nnops counterpart): the s8/u8 destination is
 * produced through the f32 epilogue instead:
 *   f = float(v) * (s_a * s_b);  r = float(C_old - zp_out) * s_out (add_to);
 *   y = act(clamp(f [+ r if residual_pre])) [+ r otherwise];
 *   q = sat(round(clamp(y / s_out, lo - zp, hi - zp)) + zp)
 * which is how an s8 add_to residual and a GELU on an integer destination are
 * defined here (nnops rejects both: linear.cpp:226).
 *
 * f32/f16 destinations (nnops' dequantizing route, DqRoute, matmul_i8.cpp:
 * 161-211; tests/reference/matmul_dq_ref.cpp:178-190):
 *   f = float(v) * (s_a * s_b) [+ bias_fp[n]] [+ C_old if add_to];
 *   y = act(clamp(f, min_clip, max_clip)), stored as f32 or f16 (nearest even);
 * `bias` must be NULL there (the fp bias is `bias_fp`, in C's type). */
typedef struct NnopsGemmI8Args {
    const void* a;
    const int8_t* b;
    const int32_t* bias;        /* [N] int32, or NULL */
    void* c;
    int64_t m, n, k;
    int64_t lda, ldb, ldc;      /* row strides in elements */
    int32_t trans_a, trans_b, a_u8;
    const float* s_a; float s_a_scalar; const int32_t* zp_a; int32_t zp_a_scalar;
    const float* s_b; float s_b_scalar; const int32_t* zp_b; int32_t zp_b_scalar;
    const float* s_out_rows; const int32_t* zp_out_rows; float s_out; int32_t zp_out;
    int32_t out_kind;           /* NNOPS_OUT_S32 / S8 / U8 */
    int32_t act;                /* NNOPS_ACT_* (integer route: NONE or RELU) */
    int32_t round_even;
    int32_t float_ep;
    float min_clip, max_clip;   /* float epilogue and f32/f16 destinations */
    int32_t add_to, residual_pre; /* float epilogue and f32/f16 destinations */
    const void* bias_fp;        /* [N] f32 or f16 (C's type), f32/f16 destinations only */
    float act_alpha, act_beta;  /* LeakyRelu / Elu alpha, HardSwish beta */
    const int32_t* b_col_sums;  /* [N] sum over k of B[k,n] (a prepacked B carries them), or
                                   NULL: computed into the workspace when the A zero point
                                   or a u8 A needs them */
} NnopsGemmI8Args;

size_t nnops_hip_gemm_i8_workspace_size(const NnopsGemmI8Args* args);
int nnops_hip_gemm_i8(const NnopsGemmI8Args* args, void* workspace, size_t workspace_bytes,
                      void* stream);

/* No counterpart in nnops. nnops_hip_gemm_i8 for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): the same kernels and results, with the workspace taken from a
 * fixed device array of NNOPS_HIP_NOALLOC_SCRATCH_BYTES that the library
 * holds on each GPU it runs on until the process ends. A call whose plan needs
 * more (nnops_hip_gemm_i8_workspace_size > the limit, e.g. a raw [K,N] B of
 * 64 MiB that is staged transposed) returns NNOPS_OUT_OF_MEMORY and enqueues
 * nothing. Calls on one GPU share the array: calls that may overlap on one
 * GPU (two streams, two threads) race. `stream` must belong to the current
 * device. Nothing is allocated, no host sync. */
#define NNOPS_HIP_NOALLOC_SCRATCH_BYTES (64u << 20)
int nnops_hip_gemm_i8_noalloc(const NnopsGemmI8Args* args, void* stream);

/* Prepacked s8 B for the HIP kernels (nnops' MatMul::prepackWeights,
 * src/ops/matmul.cpp:96-141, with a gfx950 layout in place of the CPU
 * panels). From B [K,N] (trans_b = 0) or [N,K] (trans_b = 1), row stride ldb,
 * it writes:
 *   rows   [N][kp] k-contiguous, kp = K rounded up to 128, zero padded;
 *   sums   int32 [N] = sum over k of B[k,n], at byte offset
 *          align_up(N * kp, 256).
 * A call then passes b = out, ldb = kp, trans_b = 1, b_col_sums = out + that
 * offset: every route reads the weight k-contiguous and 16-byte aligned (no
 * per-call transpose, no column-sum pass). `out` must be 256-byte aligned and
 * hold nnops_hip_prepack_i8_bytes(k, n) bytes. Stream-ordered, no allocation. */
size_t nnops_hip_prepack_i8_bytes(int64_t k, int64_t n);
int nnops_hip_prepack_i8(const int8_t* b, int64_t k, int64_t n, int64_t ldb, int32_t trans_b, void* out,
                         void* stream);

/* Prepacked Q4_1 B with blocks along N (nnops' MatMul::prepackWeights,
 * src/ops/matmul.cpp:96-141; the CPU path packs no Q4_1 form,
 * matmul_helper.cpp:695-723, this is the gfx950 one). From B [K][ceil(N/32)]
 * blocks (trans_b = 0), row pitch ldb_bytes, it writes the same blocks as
 * two planes, structure of arrays, one block column (32 columns) after
 * another:
 *   nibbles  k-blocked: block column j is kg * 128 bytes (kg = ceil(K/8)),
 *            per group of 8 rows, per nibble dword d, the 8 rows' dwords:
 *            dword d of row k, block j at byte
 *            (j * kg + k / 8) * 128 + 32 d + 4 (k % 8) (rows past K zero);
 *   d|m      block column j is kdm u32 (kdm = K rounded up to 64), row k's
 *            (f16 d low, f16 m high) at j * kdm + k (rows past K zero), the
 *            plane at byte offset align_up(nbn * kg * 128, 256);
 * nbn = ceil(N / 32). A call then passes b = out, ldb_bytes = kg * 128,
 * b_soa = 1, b_dm = out + that offset, ldb_dm = kdm: a block column's bytes
 * are two contiguous runs over the whole of K, so the GEMV streams each as
 * whole lines with no K split, and the GEMM's lane loads are contiguous 4-
 * and 16-byte runs instead of 20-byte strides. Blocks along K (trans_b = 1)
 * already stream as whole rows and have no packed form (NNOPS_UNSUPPORTED). `out` must be 256-byte aligned and hold
 * nnops_hip_prepack_q4_1_bytes(k, n) bytes. Stream-ordered, no allocation. */
size_t nnops_hip_prepack_q4_1_bytes(int64_t k, int64_t n);
int nnops_hip_prepack_q4_1(const uint8_t* b, int64_t k, int64_t n, int64_t ldb_bytes, int32_t trans_b, void* out,
                           void* stream);

/* Q4_1 codec over rows x cols values (each row its own run of blocks; a
 * partial last block takes d and m from the values that exist and leaves the
 * missing nibbles zero).
 * nnops_hip_q4_1_quantize replaces quantize_q4 (include/nnops/detail/q4_1.hpp:
 *   92-149, llama.cpp's quantize_row_q4_1_ref): src f32 (src_f16 = 0) or f16,
 *   row stride ld_src elements -> dst rows of ceil(cols / 32) 20-byte blocks,
 *   ld_dst_bytes apart (a multiple of 4, 4-byte-aligned dst). Byte-identical to
 *   the reference: d = (max - min) / 15, m = min (f16, nearest even),
 *   q = min(trunc((x - min) * (1 / d) + 0.5), 15).
 * nnops_hip_q4_1_dequantize replaces pack_q4 (q4_1.hpp:155-183): blocks ->
 *   f32 / f16 (dst_f16) rows, ld_dst elements apart; y = d * q + m in f32, f16
 *   rounded to nearest even.
 * Stream-ordered, no allocation, no workspace. */
int nnops_hip_q4_1_quantize(const void* src, int32_t src_f16, int64_t rows, int64_t cols, int64_t ld_src,
                            void* dst, int64_t ld_dst_bytes, void* stream);
int nnops_hip_q4_1_dequantize(const void* src, int64_t ld_src_bytes, int64_t rows, int64_t cols, void* dst,
                              int32_t dst_f16, int64_t ld_dst, void* stream);

/* Q4_1-weight GEMM  C[M,N] = A[M,K] x dequant(B).
 * Replaces nnops' fp x q4_1 route: matmul_qblock_fused (small M,
 * src/backend/cpu/matmul/matmul_qblock_fused.cpp:174-197) and FpRoute with
 * the Q4_1 RHS pack (matmul_helper.cpp:408-497). B is a stream of llama.cpp
 * Q4_1 blocks (20 bytes: f16 d, f16 m, 16 nibble bytes, value = d*q + m;
 * include/nnops/detail/q4_1.hpp:5-18):
 *   trans_b = 1: [N] rows of ceil(K/32) blocks along K (Linear / GGUF form),
 *   trans_b = 0: [K] rows of ceil(N/32) blocks along N,
 * consecutive rows ldb_bytes apart. A is f16 or f32 (a_f16), C is f32 or f16
 * (out_kind NNOPS_OUT_F32 / NNOPS_OUT_F16). Accumulation is f32. */
typedef struct NnopsGemmQ41Args {
    const void* a;
    const uint8_t* b;
    void* c;
    int64_t m, n, k;
    int64_t lda, ldc;           /* elements */
    int64_t ldb_bytes;
    int32_t trans_b, a_f16;
    int32_t out_kind;           /* NNOPS_OUT_F32 / NNOPS_OUT_F16 */
    /* b_soa = 1: B is the prepacked blocks-along-N form (trans_b = 0) of
     * nnops_hip_prepack_q4_1: b = the k-blocked nibble plane (ldb_bytes =
     * its block-column pitch, exactly ceil(K/8) * 128), b_dm = the d|m plane
     * (ldb_dm = its block-column pitch in u32, exactly K rounded up to 64). */
    int32_t b_soa;
    const uint32_t* b_dm;
    int64_t ldb_dm;
} NnopsGemmQ41Args;

size_t nnops_hip_gemm_q4_1_workspace_size(const NnopsGemmQ41Args* args);
int nnops_hip_gemm_q4_1(const NnopsGemmQ41Args* args, void* workspace, size_t workspace_bytes,
                        void* stream);

/* Dense fp product of nnops' float MatMul / Linear routes: C = alpha (A B)
 * for f32 x f32 or f16 x f16 (in_f16), accumulated in f32 and rounded once
 * to C's type (f32, or f16 with out_f16). Replaces the product of nnops'
 * matmul_small_fp / FpRoute<T> over dense operands
 * (src/backend/cpu/matmul/matmul_small.cpp:325-360, matmul.cpp:57-198),
 * whose f16 form keeps its accumulator in C between 128-deep k blocks; the
 * bias, beta, residual and epilogue are the output pass below.
 * A [M][lda], B [N][ldb] (trans_b) or [K][ldb], C [M][ldc]; pitches in
 * elements. The workspace holds K-split partials (small M, [K][N] B), a
 * transposed [K][N] f16 B and the ring GEMM's split partials (large f16
 * shapes): nnops_hip_gemm_fp_workspace_size bytes, 16-byte aligned. */
typedef struct NnopsGemmFpArgs {
    const void* a;
    const void* b;
    void* c;
    int64_t m, n, k;
    int64_t lda, ldb, ldc;      /* elements */
    int32_t trans_b;
    int32_t in_f16;             /* A and B f16 (else f32) */
    int32_t out_f16;            /* C f16 (else f32) */
    float alpha;
} NnopsGemmFpArgs;

size_t nnops_hip_gemm_fp_workspace_size(const NnopsGemmFpArgs* args);
int nnops_hip_gemm_fp(const NnopsGemmFpArgs* args, void* workspace, size_t workspace_bytes, void* stream);

/* Output pass of the fp x q4_1 routes over the GEMM's f32 results:
 * bias, the residual (add_to) and the epilogue (clip, activation), and the
 * gated combine of Linear's gated form. Replaces the fp epilogue of nnops'
 * FpRoute / matmul_qblock_fused output (apply_epilogue,
 * src/backend/cpu/simd_kernel/simd_epilogue.hpp:56-90; Linear's residual
 * order, src/backend/cpu/matmul/linear.cpp:276-301) and linear_gated_impl +
 * gated_combine_act (src/backend/cpu/matmul/linear.cpp:84-170, the combine
 * of src/backend/cpu/common/gate_combine.hpp:47-85).
 *   not gated:  f = src[r][c] + bias[c] (+ old if residual_pre);
 *               f = act(clip(f)); out = f (+ old, after the output type's
 *               rounding of f, if add_to and not residual_pre)
 *   matmul_order (MatMul's C = act(clip(alpha P + bias + beta C_old)),
 *               include/nnops/ops/matmul.hpp:5-11, with the accumulator
 *               init of matmul_qblock_fused.cpp:106-142): b = residual_pre
 *               ? 1 : beta; init = T(b old + bias) with a bias, else
 *               T(b old) (old itself when b = 1, 0 when b = 0), T the
 *               output type; out = act(clip(alpha src + init)). add_to is
 *               not read in this order.
 *   gated:      src holds 2n columns, gate [0, n) and value [n, 2n):
 *               g = T(src[r][c] + bias[c]), v = T(src[r][n + c] + bias[n + c])
 *               (T the output type: the reference's GEMM tile is of X's
 *               type), both clamped to +-gate_limit when finite;
 *               y = act(clip(gate_act(g) * (v + gate_beta))), out = y (+ old
 *               if add_to, after y's rounding to the output type); gate_act:
 *               Silu g / (1 + exp(-gate_alpha g)), Gelu
 *               (tanh form), Relu, Sigmoid, Tanh, None.
 * bias is in the output's type (f32 or f16), or NULL. Stream-ordered, no
 * allocation. */
typedef struct NnopsFpOutArgs {
    const float* src;           /* [rows][ld_src] f32 */
    int64_t ld_src;             /* elements */
    void* out;                  /* [rows][ld_out] f32 or f16 (out_f16) */
    int64_t ld_out;             /* elements */
    int64_t rows, n;            /* output columns n (gated: src has 2n) */
    int32_t out_f16;
    const void* bias;           /* [n], gated [2n], or NULL */
    int32_t act;                /* NNOPS_ACT_* */
    float act_alpha, act_beta, min_clip, max_clip;
    int32_t add_to, residual_pre;
    int32_t gated;
    int32_t gate_act;           /* NNOPS_ACT_NONE/RELU/GELU/SIGMOID/TANH/SILU */
    float gate_alpha, gate_beta, gate_limit;
    int32_t matmul_order;       /* 0: the orders above; 1: MatMul's (alpha, beta) */
    float alpha, beta;          /* read only when matmul_order */
} NnopsFpOutArgs;

int nnops_hip_fp_output_pass(const NnopsFpOutArgs* args, void* stream);

/* The Q4_1 GEMM with its output pass fused into the write-back: the product
 * of `g` (its c, ldc and out_kind unused) goes through `pass` (src and
 * ld_src unused; rows = g->m, n = g->n, or g->n / 2 for the gated form, whose
 * weight holds the gate rows and then the value rows) straight to pass->out,
 * with the same operations and rounding as nnops_hip_gemm_q4_1 into f32
 * followed by nnops_hip_fp_output_pass (nnops' Linear write-back,
 * src/backend/cpu/matmul/linear.cpp:74-170,233-282). Taken by the gated
 * form on the blocks-along-K ring route (trans_b, f16 A, K % 64 == 0,
 * 16-byte A rows, M past the GEMV and skinny shapes), where it saves the
 * f32 staging of both halves; NNOPS_UNSUPPORTED otherwise (the plain pass
 * included: in the write-back it costs more than its staging), with nothing
 * launched, and the caller runs the two-step form. No workspace. */
int nnops_hip_gemm_q4_1_fused(const NnopsGemmQ41Args* g, const NnopsFpOutArgs* pass, void* stream);

/* QuantizeLinear / DequantizeLinear over a rows x cols view (row strides in
 * elements), and the activation quantization of the fp-activation int8 MatMul.
 * Replaces nnops' quantize_linear_impl / dequantize_linear_impl
 * (src/backend/cpu/quant_linear.cpp:77-331) and quantize_activation in
 * matmul_dq (src/backend/cpu/matmul/matmul_i8.cpp:400-446).
 *
 * Parameter of flat element i = r * cols + c: entry (i / inner) % dim of
 * `scale` (f32) / `zero_point` (s8, u8 or s32 per zp_kind); dim <= 1 uses
 * entry 0 (NULL tables: the scalars). PerTensor: dim = 1; PerToken:
 * inner = cols, dim = rows; PerChannel(axis): inner = prod(shape[axis+1:]),
 * dim = shape[axis] (include/nnops/ops/quant_linear.hpp resolve rules).
 *   quantize    x f32/f16 -> y s8/u8:  clamp(rint(fma(x, 1/s, zp))), ties even;
 *               NaN / |v| >= 2^31 -> qmin (the x86 integer indefinite);
 *   dequantize  x s8/u8 -> y f32/f16:  fma(q, s, -zp*s) on each segment's whole
 *               16-element blocks, (q - zp) * s on its last segment % 16
 *               elements, as nnops' vector body and scalar tail
 *               (src/backend/cpu/x86_64/quant.hpp:298-340); `segment` is the
 *               reference's row: numel, cols or inner for the three modes. */
typedef struct NnopsQdqArgs {
    const void* x;
    void* y;
    int64_t rows, cols;
    int64_t ld_x, ld_y;         /* elements */
    int32_t x_kind, y_kind;     /* NNOPS_OUT_F32 / F16 / S8 / U8 */
    int32_t zp_kind;            /* NNOPS_OUT_S8 / U8 / S32: zero_point's element type */
    const float* scale;
    const void* zero_point;
    float scale_scalar;
    int32_t zp_scalar;
    int64_t inner, dim;
    int64_t segment;            /* dequantize only */
} NnopsQdqArgs;

int nnops_hip_quantize_linear(const NnopsQdqArgs* args, void* stream);
int nnops_hip_dequantize_linear(const NnopsQdqArgs* args, void* stream);

/* Library version and build target, for the caller's diagnostics. */
const char* nnops_hip_build_info(void);

/* Kernel timing for benchmarks (no counterpart in nnops; for callers that
 * measure the library, such as bench.py). Arms the calling thread's next
 * kernel launch by this library: that one launch carries `start` and `stop`
 * (hipEvent_t, created with timing enabled) on its own dispatch packet, so
 * hipEventElapsedTime(start, stop) is the kernel's execution alone, without
 * the dispatch gap an event pair recorded around the call would include.
 * One-shot: the next launch disarms it. A call that launches several kernels
 * times its first. Returns NNOPS_OK; NNOPS_INVALID_ARGUMENT if exactly one of
 * the two events is null; (null, null) disarms. */
int nnops_hip_time_next_launch(void* start_event, void* stop_event);


#ifdef __cplusplus
}
#endif

#endif /* NNOPS_AMD_H */
