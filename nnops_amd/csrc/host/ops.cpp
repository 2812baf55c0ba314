// MatMul / Linear front end for Backend::HIP: descriptor rules, workspace
// planning and the lowering of a call onto the C ABI entry points
// (nnops_hip_gemm_i8 / nnops_hip_gemm_q4_1).
//
// Follows nnops' operator front end: output-descriptor rules of
// src/ops/matmul.cpp:49-58 and src/ops/linear.cpp:29-47, validate()'s count /
// rank / K-agreement checks (src/ops/matmul.cpp:60-94), QuantParams routing of
// src/backend/cpu/matmul/matmul_tile_impl.h:366-421 (A per-token scale and zero
// point, B per-channel, output per-tensor or the epilogue's per-row
// Requantize table), batch broadcasting over the leading dims.
#include "nnops/ops/linear.hpp"
#include "nnops/ops/matmul.hpp"
#include "nnops_amd.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cstring>
#include <limits>

namespace nnops {
namespace {

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

Status from_code(int c)
{
    switch (c) {
    case NNOPS_OK: return Status::ok;
    case NNOPS_INVALID_ARGUMENT: return Status::invalid_argument;
    case NNOPS_UNSUPPORTED: return Status::unsupported;
    case NNOPS_NOT_INITIALIZED: return Status::not_initialized;
    case NNOPS_OUT_OF_MEMORY: return Status::out_of_memory;
    default: return Status::internal;
    }
}

// ---------------------------------------------------------------------------
// Problem geometry shared by MatMul and Linear.
// ---------------------------------------------------------------------------
struct Geometry {
    int64_t m = 0, n = 0, k = 0;
    int64_t batch = 1;
    bool trans_a = false, trans_b = false;
    bool b_packed = false;  // B is a PackedBHip blob (described as [N, K])
    // leading (batch) dims, broadcast
    int64_t nd = 0;
    int64_t out_batch[TensorDesc::kMaxRank]{};
    int64_t a_batch[TensorDesc::kMaxRank]{};
    int64_t b_batch[TensorDesc::kMaxRank]{};
};

/// MatMul geometry: A [..., M, K] (trans_a: [..., K, M]), B [..., K, N]
/// (trans_b: [..., N, K]); a q4_1 B's innermost dim counts values, not blocks.
Status matmul_geometry(const TensorDesc& a, const TensorDesc& b, bool ta, bool tb, Geometry& g)
{
    if (a.rank < 2 || b.rank < 2) {
        return Status::invalid_argument;
    }
    const int64_t am = a.dims[static_cast<size_t>(a.rank - 2)];
    const int64_t ak = a.dims[static_cast<size_t>(a.rank - 1)];
    const int64_t b0 = b.dims[static_cast<size_t>(b.rank - 2)];
    const int64_t b1 = b.dims[static_cast<size_t>(b.rank - 1)];
    g.trans_a = ta;
    g.trans_b = tb;
    g.m = ta ? ak : am;
    g.k = ta ? am : ak;
    if (b.layout == TensorLayout::PackedBHip) {
        // A packed B is described as [N, K] with a row pitch that makes N rows
        // cover the whole blob (prepack_s8 / prepack_q4_1 below): K must be
        // A's exactly (the column-sum and d|m plane offsets depend on it) and
        // the blob large enough for it (nnops: the backend's numel check,
        // matmul.cpp:84-90). s8: [N][kp] rows (read as transposed); q4_1: the
        // two planes of a blocks-along-N weight (read as [K, N])
        if (b.rank != 2 || b1 != g.k) {
            return Status::invalid_argument;
        }
        const int64_t unit = static_cast<int64_t>(data_type_stride_unit(b.dtype));
        const int64_t pitch = b.row_stride_elems > 0 ? b.row_stride_elems * unit
                                                     : static_cast<int64_t>(data_type_row_bytes(b.dtype, b1));
        if (b.dtype == DataType::s8) {
            if (b0 * pitch < static_cast<int64_t>(nnops_hip_prepack_i8_bytes(g.k, b0))) {
                return Status::invalid_argument;
            }
            g.trans_b = true;
        } else if (b.dtype == DataType::q4_1) {
            if (b0 * pitch < static_cast<int64_t>(nnops_hip_prepack_q4_1_bytes(g.k, b0))) {
                return Status::invalid_argument;
            }
            g.trans_b = false;
        } else {
            return Status::invalid_argument;
        }
        g.n = b0;
        g.b_packed = true;
    } else {
        const int64_t kb = tb ? b1 : b0;
        g.n = tb ? b0 : b1;
        if (kb != g.k) {
            return Status::invalid_argument;
        }
    }
    g.nd = std::max(a.rank, b.rank) - 2;
    g.batch = 1;
    for (int64_t i = 0; i < g.nd; ++i) {
        const int64_t ai = i - (g.nd - (a.rank - 2));
        const int64_t bi = i - (g.nd - (b.rank - 2));
        const int64_t da = ai >= 0 ? a.dims[static_cast<size_t>(ai)] : 1;
        const int64_t db = bi >= 0 ? b.dims[static_cast<size_t>(bi)] : 1;
        if (da != db && da != 1 && db != 1) {
            return Status::invalid_argument;
        }
        g.a_batch[i] = da;
        g.b_batch[i] = db;
        g.out_batch[i] = std::max(da, db);
        g.batch *= g.out_batch[i];
    }
    return Status::ok;
}

// ---------------------------------------------------------------------------
// Host vs device tables. QuantParams / Epilogue tables may be host arrays
// (staged into the workspace, as nnops' CUDA backend stages them) or device
// arrays (read in place).
// ---------------------------------------------------------------------------
bool is_device_pointer(const void* p)
{
    if (p == nullptr) {
        return false;
    }
    hipPointerAttribute_t attr;
    std::memset(&attr, 0, sizeof(attr));
    const hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged ||
           attr.type == hipMemoryTypeArray;
}

struct Stager {
    char* base = nullptr;
    size_t used = 0, cap = 0;
    hipStream_t stream = nullptr;
    bool ok = true;

    template <class T>
    const T* stage(const T* p, int64_t count)
    {
        if (p == nullptr || count <= 0 || is_device_pointer(p)) {
            return p;
        }
        const size_t bytes = align_up(static_cast<size_t>(count) * sizeof(T));
        if (base == nullptr || used + bytes > cap) {
            ok = false;
            return p;
        }
        char* dst = base + used;
        used += bytes;
        if (hipMemcpyAsync(dst, p, static_cast<size_t>(count) * sizeof(T), hipMemcpyHostToDevice,
                           stream) != hipSuccess) {
            ok = false;
        }
        return reinterpret_cast<const T*>(dst);
    }
};

/// Staging bytes a call may need: A's per-token scale / zero point (one entry
/// per global row of A, `a_rows`), the epilogue's per-row output table (`m`)
/// and B's per-column tables (`n`).
size_t staging_bytes(int64_t a_rows, int64_t m, int64_t n)
{
    return 2 * align_up(static_cast<size_t>(a_rows) * 4) + 2 * align_up(static_cast<size_t>(m) * 4) +
           2 * align_up(static_cast<size_t>(n) * 4);
}

/// Read a scalar that may sit in host or device memory; device memory is not
/// read from the host (that would synchronise), so it reports failure.
bool host_scalar(const float* p, float& out)
{
    if (is_device_pointer(p)) {
        return false;
    }
    out = *p;
    return true;
}
bool host_scalar(const int32_t* p, int32_t& out)
{
    if (is_device_pointer(p)) {
        return false;
    }
    out = *p;
    return true;
}

// ---------------------------------------------------------------------------
// The quantized call, independent of MatMul vs Linear.
// ---------------------------------------------------------------------------
struct QuantCall {
    bool trans_a = false, trans_b = false;
    Epilogue ep{};
    bool add_to = false, residual_pre = false;
    bool round_even = false, float_ep = false;
    bool bias = false;                  // a bias input is present
    // Linear's gated form (the weight's 2N rows: gate, then value)
    bool gated = false;
    EpilogueActivateType gate_act = EpilogueActivateType::Silu;
    float gate_alpha = 1.0f, gate_beta = 0.0f, gate_limit = std::numeric_limits<float>::infinity();
    // MatMul's product scale and old-C scale (the fp routes read them, the
    // integer routes ignore them: include/nnops/ops/matmul.hpp:37-44)
    bool matmul = false;
    float alpha = 1.0f, beta = 0.0f;

    /// The fp x q4_1 route writes its f32 results to the workspace and runs
    /// nnops_hip_fp_output_pass when there is anything after the GEMM.
    bool q4_1_pass() const
    {
        return bias || add_to || gated || epilogue_is_active(ep) || (matmul && (alpha != 1.0f || beta != 0.0f));
    }
};

int32_t out_kind_of(DataType dt)
{
    switch (dt) {
    case DataType::s32: return NNOPS_OUT_S32;
    case DataType::s8: return NNOPS_OUT_S8;
    case DataType::u8: return NNOPS_OUT_U8;
    case DataType::f32: return NNOPS_OUT_F32;
    case DataType::f16: return NNOPS_OUT_F16;
    default: return -1;
    }
}

/// Matrices of A (the product of its own batch dims, before broadcasting).
int64_t a_matrices(const Geometry& g)
{
    int64_t c = 1;
    for (int64_t i = 0; i < g.nd; ++i) {
        c *= g.a_batch[i];
    }
    return c;
}

/// Entries a per-token A table must hold: nnops indexes it by A's global row,
/// row_base + m with row_base = (A's batch offset) / (A's row stride), on the
/// dequantizing routes (src/backend/cpu/matmul/matmul_tile_impl.h:455-462).
int64_t a_table_rows(const Geometry& g)
{
    const int64_t rows_per = g.trans_a ? g.k : g.m;
    return (a_matrices(g) - 1) * rows_per + g.m;
}

/// Row pitch of a PackedBHip blob for a K (nnops_hip_prepack_i8's layout).
int64_t packed_pitch(int64_t k)
{
    return (k + 127) / 128 * 128;
}

bool is_fp_quant_pair(DataType a, DataType b)
{
    return (a == DataType::f32 || a == DataType::f16) && b == DataType::s8;
}

/// nnops' dense float pairs: f32 x f32 and f16 x f16 (the output follows A).
bool is_dense_fp_pair(DataType a, DataType b)
{
    return (a == DataType::f32 || a == DataType::f16) && b == a;
}

NnopsGemmFpArgs fp_args_from_geometry(const Geometry& g, bool f16, bool out_f16)
{
    NnopsGemmFpArgs x{};
    x.m = g.m;
    x.n = g.n;
    x.k = g.k;
    x.trans_b = g.trans_b;
    x.in_f16 = f16;
    x.out_f16 = out_f16;
    x.lda = g.k;
    x.ldb = g.trans_b ? g.k : g.n;
    x.ldc = g.n;
    x.alpha = 1.0f;
    return x;
}

NnopsGemmI8Args i8_args_from_geometry(const Geometry& g, int32_t out_kind)
{
    NnopsGemmI8Args x{};
    x.m = g.m;
    x.n = g.n;
    x.k = g.k;
    x.trans_a = g.trans_a;
    x.trans_b = g.trans_b;
    x.lda = g.trans_a ? g.m : g.k;
    x.ldb = g.b_packed ? packed_pitch(g.k) : (g.trans_b ? g.k : g.n);
    x.ldc = g.n;
    x.out_kind = out_kind;
    return x;
}

NnopsGemmQ41Args q41_args_from_geometry(const Geometry& g, const QuantCall& q, int32_t out_kind)
{
    NnopsGemmQ41Args x{};
    x.m = g.m;
    x.n = g.n;
    x.k = g.k;
    (void)q;
    x.trans_b = g.trans_b;
    x.a_f16 = 1;
    x.lda = g.k;
    x.ldc = g.n;
    x.ldb_bytes = static_cast<int64_t>(data_type_row_bytes(DataType::q4_1, g.trans_b ? g.k : g.n));
    x.out_kind = out_kind;
    if (g.b_packed) {
        // the planes of nnops_hip_prepack_q4_1, one block column after
        // another: ceil(K/8) * 128 nibble bytes and K rounded up to 64 d|m
        // dwords per block column (b_dm is set with the pointer)
        x.b_soa = 1;
        x.ldb_bytes = (g.k + 7) / 8 * 128;
        x.ldb_dm = (g.k + 63) / 64 * 64;
    }
    return x;
}

/// Workspace of the int8 GEMM call: staging for host-side tables, then the
/// GEMM's own partial-sum / split-K region.
size_t i8_workspace(const Geometry& g, int32_t out_kind)
{
    // The kernel plan (and so its region) depends on what a descriptor does not
    // carry: zero points, tables, pointer alignment. Size for the largest: the
    // plan of plain operands (the [K,N] column GEMV's partials), the plan with
    // zero points (a staged B^T plus K-split partials) and the plan of an
    // unaligned destination (raw partials for the reduce).
    NnopsGemmI8Args x = i8_args_from_geometry(g, out_kind);
    size_t need = nnops_hip_gemm_i8_workspace_size(&x);
    x.zp_a_scalar = 1;
    need = std::max(need, nnops_hip_gemm_i8_workspace_size(&x));
    // a destination too unaligned for the fused output passes (never
    // dereferenced by the size query): the split-partials plan
    x.c = reinterpret_cast<void*>(uintptr_t{1});
    need = std::max(need, nnops_hip_gemm_i8_workspace_size(&x));
    return staging_bytes(a_table_rows(g), g.m, g.n) + align_up(need);
}

/// The fp-activation route's own prefix: A's staged scale / zero-point tables
/// and the quantized copy A_q (compact, one byte per element).
size_t fp_quant_prefix(const Geometry& g)
{
    const int64_t rows = a_matrices(g) * g.m;
    return 2 * align_up(static_cast<size_t>(rows) * 4) + align_up(static_cast<size_t>(rows * g.k));
}

/// The f32 results of one batch matrix of the fp x q4_1 route, ahead of its
/// output pass (0 when the GEMM writes the destination directly).
size_t q4_1_pass_bytes(const Geometry& g, const QuantCall& q)
{
    return q.q4_1_pass() ? align_up(static_cast<size_t>(g.m) * static_cast<size_t>(g.n) * sizeof(float)) : 0;
}

size_t quant_workspace(const TensorDesc& a, const TensorDesc& b, const TensorDesc* out,
                       const QuantCall& q, DataType out_dtype)
{
    Geometry g;
    if (!is_ok(matmul_geometry(a, b, q.trans_a, q.trans_b, g))) {
        return 0;
    }
    if (is_int8_matmul(a.dtype, b.dtype)) {
        return i8_workspace(g, out_kind_of(out_dtype));
    }
    if (is_fp_quant_pair(a.dtype, b.dtype)) {
        if (g.trans_a) {
            return 0;
        }
        return fp_quant_prefix(g) + i8_workspace(g, out_kind_of(a.dtype));
    }
    if (is_q4_1_matmul(a.dtype, b.dtype)) {
        const DataType odt = out != nullptr ? out->dtype : a.dtype;
        NnopsGemmQ41Args x = q41_args_from_geometry(g, q, q.q4_1_pass() ? NNOPS_OUT_F32 : out_kind_of(odt));
        x.a_f16 = a.dtype == DataType::f16;
        return q4_1_pass_bytes(g, q) + align_up(nnops_hip_gemm_q4_1_workspace_size(&x));
    }
    if (is_dense_fp_pair(a.dtype, b.dtype) && !g.b_packed) {
        const NnopsGemmFpArgs x =
            fp_args_from_geometry(g, a.dtype == DataType::f16, !q.q4_1_pass() && a.dtype == DataType::f16);
        return q4_1_pass_bytes(g, q) + align_up(nnops_hip_gemm_fp_workspace_size(&x));
    }
    return 0;
}

/// Byte offset of batch index `bi` for an operand whose leading dims are
/// `dims` (broadcast against `out`), given its row pitch and the rows per
/// matrix.
int64_t batch_offset(int64_t bi, const Geometry& g, const int64_t* dims, int64_t matrix_bytes)
{
    int64_t off = 0, stride = matrix_bytes, rem = bi;
    // walk dims from innermost batch axis outward
    std::array<int64_t, TensorDesc::kMaxRank> coord{};
    for (int64_t d = g.nd - 1; d >= 0; --d) {
        coord[static_cast<size_t>(d)] = rem % g.out_batch[d];
        rem /= g.out_batch[d];
    }
    for (int64_t d = g.nd - 1; d >= 0; --d) {
        if (dims[d] != 1) {
            off += coord[static_cast<size_t>(d)] * stride;
        }
        stride *= dims[d];
    }
    return off;
}

int32_t act_code(EpilogueActivateType t)
{
    return static_cast<int32_t>(t);  // NNOPS_ACT_* share nnops' numbering
}

/// The int8 GEMM over s8/u8 A (an fp activation arrives here already
/// quantized), every destination: s32, s8/u8 requantized, f32/f16 dequantized
/// (src/backend/cpu/matmul/matmul_i8.cpp:470-494). `ws` is i8_workspace()
/// bytes: the staging tables first, then the GEMM's region.
Status run_i8(const QuantCall& q, const Geometry& g, TensorView& out, const TensorView& a,
              const TensorView& b, const TensorView* bias, hipStream_t stream, void* workspace,
              size_t ws_bytes)
{
    const int32_t ok = out_kind_of(out.data_type());
    if (ok < 0) {
        return Status::unsupported;
    }
    const bool fp_out = ok == NNOPS_OUT_F32 || ok == NNOPS_OUT_F16;
    if (bias != nullptr) {
        const DataType want = fp_out ? out.data_type() : DataType::s32;
        if (bias->data_type() != want || bias->numel() < g.n) {
            return Status::invalid_argument;
        }
    }
    if (q.add_to && ok == NNOPS_OUT_S32) {
        return Status::unsupported;
    }
    NnopsGemmI8Args x = i8_args_from_geometry(g, ok);
    x.a_u8 = a.data_type() == DataType::u8;
    x.lda = a.row_stride_elems();
    x.ldb = g.b_packed ? packed_pitch(g.k) : b.row_stride_elems();
    x.ldc = out.row_stride_elems();
    if (g.b_packed) {
        x.b_col_sums = reinterpret_cast<const int32_t*>(
            b.ptr<const char>() + align_up(static_cast<size_t>(g.n * packed_pitch(g.k))));
    }
    x.add_to = q.add_to;
    x.residual_pre = q.residual_pre;
    x.min_clip = q.ep.min_clip;
    x.max_clip = q.ep.max_clip;
    x.act_alpha = q.ep.alpha;
    x.act_beta = q.ep.beta;
    if (fp_out) {
        // dequantize -> bias -> [residual] -> clip -> activation, any activation
        x.bias_fp = bias != nullptr ? bias->ptr<const void>() : nullptr;
        x.act = act_code(q.ep.type);
    } else {
        x.bias = bias != nullptr ? bias->ptr<const int32_t>() : nullptr;
        x.round_even = q.round_even;
        x.float_ep = (q.float_ep || q.add_to) && ok != NNOPS_OUT_S32;
        switch (q.ep.type) {
        case EpilogueActivateType::None: x.act = NNOPS_ACT_NONE; break;
        case EpilogueActivateType::Relu: x.act = NNOPS_ACT_RELU; break;
        case EpilogueActivateType::Gelu: x.act = x.float_ep ? NNOPS_ACT_GELU : NNOPS_ACT_NONE; break;
        default:
            // nnops' integer pass honours only Relu and ignores the rest
            // (matmul_i8.cpp:100-103); the float epilogue has no route for them.
            if (x.float_ep) {
                return Status::unsupported;
            }
            x.act = NNOPS_ACT_NONE;
        }
        if (!x.float_ep) {
            // clip bounds are not applied on an integer destination (nnops)
            x.min_clip = -std::numeric_limits<float>::infinity();
            x.max_clip = std::numeric_limits<float>::infinity();
        }
    }

    const int64_t a_rows = a_table_rows(g);
    const size_t stage_cap = staging_bytes(a_rows, g.m, g.n);
    Stager st;
    st.base = static_cast<char*>(workspace);
    st.cap = workspace != nullptr ? std::min(ws_bytes, stage_cap) : 0;
    st.stream = stream;
    const QuantParams& qa = a.quant_params();
    const QuantParams& qb = b.quant_params();
    const QuantParams& qc = out.quant_params();
    // the dequantizing routes index A's per-token tables by global row
    x.s_a = st.stage(qa.scale_data, fp_out ? a_rows : g.m);
    x.s_a_scalar = qa.scale;
    x.zp_a = st.stage(qa.zero_point_data, fp_out ? a_rows : g.m);
    x.zp_a_scalar = qa.zero_point;
    x.s_b = st.stage(qb.scale_data, g.n);
    x.s_b_scalar = qb.scale;
    x.zp_b = st.stage(qb.zero_point_data, g.n);
    x.zp_b_scalar = qb.zero_point;
    if (!fp_out) {
        x.s_out = qc.scale;
        x.zp_out = qc.zero_point;
        if (qc.scale_data != nullptr && !host_scalar(qc.scale_data, x.s_out)) {
            return Status::unsupported;
        }
        if (qc.zero_point_data != nullptr && !host_scalar(qc.zero_point_data, x.zp_out)) {
            return Status::unsupported;
        }
        if (q.ep.quant == EpilogueQuantType::Requantize && q.ep.quant_param_count > 0) {
            if (q.ep.quant_param_count > 1) {
                if (q.ep.quant_param_count < g.m) {
                    return Status::invalid_argument;
                }
                x.s_out_rows = st.stage(q.ep.quant_scales, g.m);
                x.zp_out_rows = st.stage(q.ep.quant_zero_points, g.m);
            } else {
                if (q.ep.quant_scales != nullptr && !host_scalar(q.ep.quant_scales, x.s_out)) {
                    return Status::unsupported;
                }
                x.zp_out = 0;
                if (q.ep.quant_zero_points != nullptr && !host_scalar(q.ep.quant_zero_points, x.zp_out)) {
                    return Status::unsupported;
                }
            }
        }
    }
    if (!st.ok) {
        return Status::not_initialized;
    }
    const size_t need = nnops_hip_gemm_i8_workspace_size(&x);
    if (need > 0 && (workspace == nullptr || ws_bytes < stage_cap + need)) {
        return Status::not_initialized;
    }
    void* ws = need > 0 ? static_cast<char*>(workspace) + stage_cap : nullptr;

    const int64_t a_rows_per = g.trans_a ? g.k : g.m;
    const int64_t b_rows_per = g.trans_b ? g.n : g.k;
    const int64_t a_mat = a_rows_per * a.pitch();
    const int64_t b_mat = b_rows_per * b.pitch();
    const int64_t c_mat = g.m * out.pitch();
    for (int64_t bi = 0; bi < g.batch; ++bi) {
        NnopsGemmI8Args xb = x;
        const int64_t a_off = batch_offset(bi, g, g.a_batch, a_mat);
        xb.a = a.ptr<const char>() + a_off;
        xb.b = reinterpret_cast<const int8_t*>(b.ptr<const char>() + batch_offset(bi, g, g.b_batch, b_mat));
        xb.c = out.ptr<char>() + batch_offset(bi, g, g.out_batch, c_mat);
        if (fp_out && a.pitch() > 0) {
            const int64_t row_base = a_off / a.pitch();
            xb.s_a = x.s_a != nullptr ? x.s_a + row_base : nullptr;
            xb.zp_a = x.zp_a != nullptr ? x.zp_a + row_base : nullptr;
        }
        const int rc = nnops_hip_gemm_i8(&xb, ws, need, stream);
        if (rc != NNOPS_OK) {
            return from_code(rc);
        }
    }
    return Status::ok;
}

/// fp activations with offline per-tensor / per-token QuantParams x s8
/// weights: QuantizeLinear A into A_q (A's own parameters, ties to even), then
/// the int8 GEMM dequantizing into A's dtype
/// (src/backend/cpu/matmul/matmul_i8.cpp:334-463).
Status run_fp_quant(const QuantCall& q, const Geometry& g, DataType act_dtype, TensorView& out,
                    const TensorView& a, const TensorView& b, const TensorView* bias,
                    hipStream_t stream, void* workspace, size_t ws_bytes)
{
    const QuantParams& qa = a.quant_params();
    const bool quantized = qa.is_active() && (qa.granularity == QuantGranularity::PerTensor ||
                                              qa.granularity == QuantGranularity::PerToken);
    if (!quantized) {
        return Status::invalid_argument;
    }
    if (g.trans_a) {
        return Status::unsupported;
    }
    if (act_dtype != DataType::s8 && act_dtype != DataType::u8) {
        return Status::invalid_argument;
    }
    if (out.data_type() != a.data_type()) {
        return Status::invalid_argument;
    }
    const int64_t rows = a_matrices(g) * g.m;
    const size_t prefix = fp_quant_prefix(g);
    if (workspace == nullptr || ws_bytes < prefix) {
        return Status::not_initialized;
    }
    Stager st;
    st.base = static_cast<char*>(workspace);
    st.cap = 2 * align_up(static_cast<size_t>(rows) * 4);
    st.stream = stream;
    const float* s_tab = st.stage(qa.scale_data, rows);
    const int32_t* z_tab = st.stage(qa.zero_point_data, rows);
    if (!st.ok) {
        return Status::not_initialized;
    }
    void* aq = static_cast<char*>(workspace) + st.cap;

    NnopsQdqArgs qd{};
    qd.x = a.ptr<const void>();
    qd.y = aq;
    qd.rows = rows;
    qd.cols = g.k;
    qd.ld_x = a.row_stride_elems();
    qd.ld_y = g.k;
    qd.x_kind = out_kind_of(a.data_type());
    qd.y_kind = act_dtype == DataType::u8 ? NNOPS_OUT_U8 : NNOPS_OUT_S8;
    qd.zp_kind = NNOPS_OUT_S32;
    qd.scale = s_tab;
    qd.zero_point = z_tab;
    qd.scale_scalar = qa.scale;
    qd.zp_scalar = qa.zero_point;
    qd.inner = g.k;
    qd.dim = (s_tab != nullptr || z_tab != nullptr) ? rows : 1;
    qd.segment = g.k;
    if (const int rc = nnops_hip_quantize_linear(&qd, stream); rc != NNOPS_OK) {
        return from_code(rc);
    }

    // A_q: A's shape, compact, A's (now device-resident) parameters
    QuantParams qq = qa;
    qq.scale_data = s_tab;
    qq.zero_point_data = z_tab;
    std::array<int64_t, TensorDesc::kMaxRank> shape{};
    for (int64_t i = 0; i < a.rank(); ++i) {
        shape[static_cast<size_t>(i)] = a.shape(i);
    }
    const TensorView av(std::span<const int64_t>(shape.data(), static_cast<size_t>(a.rank())), act_dtype,
                        aq, g.k, TensorLayout::Dense, qq);
    return run_i8(q, g, out, av, b, bias, stream, static_cast<char*>(workspace) + prefix, ws_bytes - prefix);
}

/// The output pass's arguments over the f32 product staged at the head of
/// the workspace (rows x g.n, the gated form's 2N columns included).
NnopsFpOutArgs fp_pass_args(const QuantCall& q, const Geometry& g, const TensorView& out, const TensorView* bias,
                            const void* staged)
{
    NnopsFpOutArgs fo{};
    fo.src = static_cast<const float*>(staged);
    fo.ld_src = g.n;
    fo.ld_out = out.row_stride_elems();
    fo.rows = g.m;
    fo.n = q.gated ? g.n / 2 : g.n;
    fo.out_f16 = out.data_type() == DataType::f16;
    fo.bias = bias != nullptr ? bias->ptr<const void>() : nullptr;
    fo.act = static_cast<int32_t>(q.ep.type);
    fo.act_alpha = q.ep.alpha;
    fo.act_beta = q.ep.beta;
    fo.min_clip = q.ep.min_clip;
    fo.max_clip = q.ep.max_clip;
    fo.add_to = q.add_to;
    fo.residual_pre = q.residual_pre;
    fo.gated = q.gated;
    fo.gate_act = static_cast<int32_t>(q.gate_act);
    fo.gate_alpha = q.gate_alpha;
    fo.gate_beta = q.gate_beta;
    fo.gate_limit = q.gate_limit;
    fo.matmul_order = q.matmul;
    fo.alpha = q.alpha;
    fo.beta = q.beta;
    return fo;
}

Status run_quant(const QuantCall& q, TensorView& out, std::span<const TensorView> inputs,
                 const ComputeContext& ctx, void* workspace, size_t ws_bytes,
                 DataType act_dtype = DataType::s8)
{
    const TensorView& a = inputs[0];
    const TensorView& b = inputs[1];
    const TensorView* bias = inputs.size() > 2 ? &inputs[2] : nullptr;
    Geometry g;
    if (Status s = matmul_geometry(a.desc(), b.desc(), q.trans_a, q.trans_b, g); !is_ok(s)) {
        return s;
    }
    // The destination must be [..., M, N] with the broadcast batch (the
    // gated form: [..., M, N / 2]).
    const int64_t n_dst = q.gated ? g.n / 2 : g.n;
    if (out.rank() < 2 || out.shape(out.rank() - 2) != g.m || out.shape(out.rank() - 1) != n_dst ||
        out.numel() != g.batch * g.m * n_dst) {
        return Status::invalid_argument;
    }
    if (g.m == 0 || g.n == 0 || g.batch == 0) {
        return Status::ok;
    }
    hipStream_t stream = static_cast<hipStream_t>(ctx.hip_stream);
    const int64_t a_rows_per = g.trans_a ? g.k : g.m;
    const int64_t b_rows_per = g.trans_b ? g.n : g.k;

    if (is_int8_matmul(a.data_type(), b.data_type())) {
        return run_i8(q, g, out, a, b, bias, stream, workspace, ws_bytes);
    }
    if (is_fp_quant_pair(a.data_type(), b.data_type())) {
        return run_fp_quant(q, g, act_dtype, out, a, b, bias, stream, workspace, ws_bytes);
    }

    if (is_q4_1_matmul(a.data_type(), b.data_type())) {
        if (g.trans_a) {
            return Status::unsupported;
        }
        const int32_t ok = out_kind_of(out.data_type());
        if (ok != NNOPS_OUT_F32 && !(ok == NNOPS_OUT_F16 && a.data_type() == DataType::f16)) {
            return Status::unsupported;
        }
        const bool pass = q.q4_1_pass();
        if (pass) {
            // the output pass reads the bias in the destination's type
            if (bias != nullptr && (bias->data_type() != out.data_type() || bias->numel() < g.n)) {
                return Status::invalid_argument;
            }
            if (q.gated && ((g.n % 2) != 0 || out.data_type() != a.data_type())) {
                return Status::invalid_argument;
            }
        }
        NnopsGemmQ41Args x = q41_args_from_geometry(g, q, pass ? NNOPS_OUT_F32 : ok);
        x.a_f16 = a.data_type() == DataType::f16;
        x.lda = a.row_stride_elems();
        x.ldc = pass ? g.n : out.row_stride_elems();
        if (g.b_packed) {
            x.b_dm = reinterpret_cast<const uint32_t*>(
                b.ptr<const char>() + align_up(static_cast<size_t>((g.n + 31) / 32 * x.ldb_bytes)));
        } else {
            x.ldb_bytes = b.pitch();
        }
        const size_t tmp = q4_1_pass_bytes(g, q);
        const size_t need = nnops_hip_gemm_q4_1_workspace_size(&x);
        if ((need > 0 || tmp > 0) && (workspace == nullptr || ws_bytes < tmp + align_up(need))) {
            return Status::not_initialized;
        }
        char* gemm_ws = static_cast<char*>(workspace) + tmp;
        NnopsFpOutArgs fo = fp_pass_args(q, g, out, bias, workspace);
        const int64_t a_mat = a_rows_per * a.pitch();
        const int64_t b_mat = b_rows_per * b.pitch();
        const int64_t c_mat = g.m * out.pitch();
        for (int64_t bi = 0; bi < g.batch; ++bi) {
            NnopsGemmQ41Args xb = x;
            xb.a = a.ptr<const char>() + batch_offset(bi, g, g.a_batch, a_mat);
            xb.b = reinterpret_cast<const uint8_t*>(b.ptr<const char>() + batch_offset(bi, g, g.b_batch, b_mat));
            char* cb = out.ptr<char>() + batch_offset(bi, g, g.out_batch, c_mat);
            xb.c = pass ? workspace : static_cast<void*>(cb);
            if (pass) {
                // the output pass in the GEMM's write-back where its route
                // takes it, else the GEMM into the workspace and the pass
                fo.out = cb;
                const int rf = nnops_hip_gemm_q4_1_fused(&xb, &fo, stream);
                if (rf == NNOPS_OK) {
                    continue;
                }
                if (rf != NNOPS_UNSUPPORTED) {
                    return from_code(rf);
                }
            }
            const int rc = nnops_hip_gemm_q4_1(&xb, gemm_ws, need, stream);
            if (rc != NNOPS_OK) {
                return from_code(rc);
            }
            if (pass) {
                if (const int rp = nnops_hip_fp_output_pass(&fo, stream); rp != NNOPS_OK) {
                    return from_code(rp);
                }
            }
        }
        return Status::ok;
    }

    if (is_dense_fp_pair(a.data_type(), b.data_type())) {
        // nnops' float route: the output follows A; a bias of the output's type
        if (g.trans_a || g.b_packed) {
            return Status::unsupported;
        }
        if (out.data_type() != a.data_type()) {
            return Status::invalid_argument;
        }
        const bool pass = q.q4_1_pass();
        if (bias != nullptr && (bias->data_type() != out.data_type() || bias->numel() < g.n)) {
            return Status::invalid_argument;
        }
        if (q.gated && (g.n % 2) != 0) {
            return Status::invalid_argument;
        }
        const bool f16 = a.data_type() == DataType::f16;
        NnopsGemmFpArgs x = fp_args_from_geometry(g, f16, !pass && f16);
        x.lda = a.row_stride_elems();
        x.ldb = b.row_stride_elems();
        x.ldc = pass ? g.n : out.row_stride_elems();
        const size_t tmp = q4_1_pass_bytes(g, q);
        const size_t need = nnops_hip_gemm_fp_workspace_size(&x);
        if ((need > 0 || tmp > 0) && (workspace == nullptr || ws_bytes < tmp + align_up(need))) {
            return Status::not_initialized;
        }
        char* gemm_ws = static_cast<char*>(workspace) + tmp;
        NnopsFpOutArgs fo = fp_pass_args(q, g, out, bias, workspace);
        const int64_t a_mat = a_rows_per * a.pitch();
        const int64_t b_mat = b_rows_per * b.pitch();
        const int64_t c_mat = g.m * out.pitch();
        for (int64_t bi = 0; bi < g.batch; ++bi) {
            NnopsGemmFpArgs xb = x;
            xb.a = a.ptr<const char>() + batch_offset(bi, g, g.a_batch, a_mat);
            xb.b = b.ptr<const char>() + batch_offset(bi, g, g.b_batch, b_mat);
            char* cb = out.ptr<char>() + batch_offset(bi, g, g.out_batch, c_mat);
            xb.c = pass ? workspace : static_cast<void*>(cb);
            const int rc = nnops_hip_gemm_fp(&xb, gemm_ws, need, stream);
            if (rc != NNOPS_OK) {
                return from_code(rc);
            }
            if (pass) {
                fo.out = cb;
                if (const int rp = nnops_hip_fp_output_pass(&fo, stream); rp != NNOPS_OK) {
                    return from_code(rp);
                }
            }
        }
        return Status::ok;
    }
    return Status::unsupported;
}

Status check_views(std::span<TensorView> outputs, std::span<const TensorView> inputs)
{
    if (inputs.size() < 2 || inputs.size() > 3 || outputs.size() != 1) {
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

TensorDesc output_desc(const Geometry& g, DataType dt, const TensorDesc& a, const TensorDesc& b)
{
    TensorDesc d;
    d.rank = g.nd + 2;
    for (int64_t i = 0; i < g.nd; ++i) {
        d.dims[static_cast<size_t>(i)] = g.out_batch[i];
    }
    d.dims[static_cast<size_t>(g.nd)] = g.m;
    d.dims[static_cast<size_t>(g.nd + 1)] = g.n;
    d.dtype = dt;
    (void)a;
    (void)b;
    return d;
}

}  // namespace

// ===========================================================================
// MatMul
// ===========================================================================
std::unique_ptr<MatMul> MatMul::create(const MatMulAttributes& attrs, Backend backend)
{
    return std::unique_ptr<MatMul>(new MatMul(attrs, backend));
}

std::vector<TensorDesc> MatMul::getOutputTensorDesc(std::span<const TensorDesc> inputs) const
{
    if (inputs.size() < 2) {
        return {};
    }
    Geometry g;
    if (!is_ok(matmul_geometry(inputs[0], inputs[1], attrs_.transpose_a, attrs_.transpose_b, g))) {
        return {};
    }
    const DataType dt = is_int8_matmul(inputs[0].dtype, inputs[1].dtype) ? attrs_.output_dtype
                                                                         : inputs[0].dtype;
    return {output_desc(g, dt, inputs[0], inputs[1])};
}

Status MatMul::validate(std::span<const TensorDesc> inputs, std::span<const TensorDesc> outputs) const
{
    if (inputs.size() < 2 || inputs.size() > 3 || outputs.size() != 1) {
        return Status::invalid_argument;
    }
    Geometry g;
    return matmul_geometry(inputs[0], inputs[1], attrs_.transpose_a, attrs_.transpose_b, g);
}

namespace {

QuantCall matmul_call(const MatMulAttributes& attrs, bool bias)
{
    QuantCall q;
    q.trans_a = attrs.transpose_a;
    q.trans_b = attrs.transpose_b;
    q.ep = attrs.epilogue;
    q.residual_pre = attrs.residual_pre_activation;
    q.add_to = attrs.residual_pre_activation;  // MatMul's residual is the pre-activation fold
    q.round_even = attrs.requant_round_even;
    q.float_ep = attrs.float_epilogue;
    q.bias = bias;
    q.matmul = true;
    q.alpha = attrs.alpha;
    q.beta = attrs.beta;
    return q;
}

}  // namespace

size_t MatMul::getWorkspaceSize(std::span<const TensorDesc> inputs,
                                std::span<const TensorDesc> outputs) const
{
    if (inputs.size() < 2) {
        return 0;
    }
    const QuantCall q = matmul_call(attrs_, inputs.size() > 2);
    const DataType odt = !outputs.empty() ? outputs[0].dtype : attrs_.output_dtype;
    return quant_workspace(inputs[0], inputs[1], outputs.empty() ? nullptr : &outputs[0], q, odt);
}

Status MatMul::compute(std::span<TensorView> outputs, std::span<const TensorView> inputs,
                       const ComputeContext& ctx, void* workspace)
{
    if (Status s = check_views(outputs, inputs); !is_ok(s)) {
        return s;
    }
    if (backend_ != Backend::HIP) {
        return Status::unsupported;
    }
    const TensorDesc descs_in[3] = {inputs[0].desc(), inputs[1].desc(),
                                    inputs.size() > 2 ? inputs[2].desc() : TensorDesc{}};
    const TensorDesc desc_out = outputs[0].desc();
    if (Status s = validate(std::span<const TensorDesc>(descs_in, inputs.size()),
                            std::span<const TensorDesc>(&desc_out, 1));
        !is_ok(s)) {
        return s;
    }
    if (is_int8_matmul(inputs[0].data_type(), inputs[1].data_type()) &&
        outputs[0].data_type() != attrs_.output_dtype) {
        return Status::invalid_argument;
    }
    const QuantCall q = matmul_call(attrs_, inputs.size() > 2);
    const size_t ws = getWorkspaceSize(std::span<const TensorDesc>(descs_in, inputs.size()),
                                       std::span<const TensorDesc>(&desc_out, 1));
    return run_quant(q, outputs[0], inputs, ctx, workspace, workspace != nullptr ? ws : 0,
                     attrs_.act_quant_dtype);
}

// ===========================================================================
// Linear
// ===========================================================================
std::unique_ptr<Linear> Linear::create(const LinearAttributes& attrs, Backend backend)
{
    return std::unique_ptr<Linear>(new Linear(attrs, backend));
}

namespace {

// Linear's X [..., K] flattened to [rows, K]; W [N, K] (q4_1: K in blocks).
bool linear_descs(std::span<const TensorDesc> inputs, TensorDesc& x2, TensorDesc& w)
{
    if (inputs.size() < 2 || inputs[0].rank < 1 || inputs[1].rank != 2) {
        return false;
    }
    const TensorDesc& x = inputs[0];
    x2 = TensorDesc{};
    x2.rank = 2;
    x2.dims[0] = x.rank >= 2 ? x.rows() : 1;
    x2.dims[1] = x.cols();
    x2.dtype = x.dtype;
    x2.row_stride_elems = x.row_stride_elems;
    w = inputs[1];
    return true;
}

DataType linear_out_dtype(const LinearAttributes& attrs, DataType x, DataType w)
{
    if (is_int8_matmul(x, w)) {
        const DataType o = attrs.output_dtype;
        const bool known = o == DataType::f16 || o == DataType::f32 || o == DataType::s32 ||
                           o == DataType::s8 || o == DataType::u8;
        return known ? o : DataType::f32;
    }
    return x;
}

/// Linear's call: the residual folds into the GEMM in the pre-activation
/// order, and an identity epilogue folds either way
/// (src/backend/cpu/matmul/linear.cpp:276-282); the gated form's combine adds
/// it after its own epilogue.
QuantCall linear_call(const LinearAttributes& attrs, bool bias)
{
    QuantCall q;
    q.trans_b = true;
    q.ep = attrs.epilogue;
    q.add_to = attrs.add_to;
    q.residual_pre = attrs.add_to && !attrs.gated &&
                     (attrs.residual_pre_activation || !epilogue_is_active(attrs.epilogue));
    q.round_even = attrs.requant_round_even;
    q.float_ep = attrs.float_epilogue;
    q.bias = bias;
    q.gated = attrs.gated;
    q.gate_act = attrs.gate_activation;
    q.gate_alpha = attrs.gate_alpha;
    q.gate_beta = attrs.gate_beta;
    q.gate_limit = attrs.gate_limit;
    return q;
}

}  // namespace

std::vector<TensorDesc> Linear::getOutputTensorDesc(std::span<const TensorDesc> inputs) const
{
    TensorDesc x2, w;
    if (!linear_descs(inputs, x2, w)) {
        return {};
    }
    TensorDesc d = inputs[0];
    d.dims[static_cast<size_t>(d.rank - 1)] = attrs_.gated ? w.dims[0] / 2 : w.dims[0];
    d.dtype = linear_out_dtype(attrs_, inputs[0].dtype, w.dtype);
    d.row_stride_elems = 0;
    return {d};
}

Status Linear::validate(std::span<const TensorDesc> inputs, std::span<const TensorDesc> outputs) const
{
    if (inputs.size() < 2 || inputs.size() > 3 || outputs.size() != 1) {
        return Status::invalid_argument;
    }
    TensorDesc x2, w;
    if (!linear_descs(inputs, x2, w)) {
        return Status::invalid_argument;
    }
    if (attrs_.gated) {
        // nnops' gated form (src/ops/linear.cpp:63-107): Silu / Gelu / Relu /
        // Sigmoid / Tanh / None, no pre-activation residual, W [2N, K], bias
        // [2N] of X's type, output [..., N]: over a dense weight of X's type
        // (nnops' rule, src/ops/linear.cpp:92), and here also over a q4_1
        // weight (blocks along K, the Linear form).
        if (attrs_.add_to && attrs_.residual_pre_activation) {
            return Status::unsupported;
        }
        switch (attrs_.gate_activation) {
        case EpilogueActivateType::Silu:
        case EpilogueActivateType::Gelu:
        case EpilogueActivateType::Relu:
        case EpilogueActivateType::Sigmoid:
        case EpilogueActivateType::Tanh:
        case EpilogueActivateType::None:
            break;
        default:
            return Status::unsupported;
        }
        if ((x2.dtype != DataType::f32 && x2.dtype != DataType::f16) ||
            (w.dtype != DataType::q4_1 && w.dtype != x2.dtype) || w.layout != TensorLayout::Dense) {
            return Status::unsupported;
        }
        if (w.dims[0] <= 0 || (w.dims[0] % 2) != 0) {
            return Status::invalid_argument;
        }
        if (inputs.size() > 2 && (inputs[2].dtype != x2.dtype || inputs[2].numel() != w.dims[0])) {
            return Status::invalid_argument;
        }
        if (!outputs.empty() && outputs[0].rank >= 1 &&
            (outputs[0].dims[static_cast<size_t>(outputs[0].rank - 1)] != w.dims[0] / 2 ||
             outputs[0].dtype != x2.dtype)) {
            return Status::invalid_argument;
        }
    }
    if (w.layout == TensorLayout::PackedBHip) {
        // [N, K] with a pitch covering the blob (prepack_s8)
        const int64_t pitch = w.row_stride_elems > 0 ? w.row_stride_elems : w.dims[1];
        if (w.dtype != DataType::s8 || w.dims[1] != x2.dims[1] ||
            w.dims[0] * pitch < static_cast<int64_t>(nnops_hip_prepack_i8_bytes(x2.dims[1], w.dims[0]))) {
            return Status::invalid_argument;
        }
    } else if (x2.dims[1] != w.dims[1]) {
        return Status::invalid_argument;
    }
    if (inputs.size() > 2 && inputs[2].numel() != w.dims[0]) {
        return Status::invalid_argument;
    }
    return Status::ok;
}

size_t Linear::getWorkspaceSize(std::span<const TensorDesc> inputs,
                                std::span<const TensorDesc> outputs) const
{
    TensorDesc x2, w;
    if (!linear_descs(inputs, x2, w)) {
        return 0;
    }
    const QuantCall q = linear_call(attrs_, inputs.size() > 2);
    const DataType odt = !outputs.empty() ? outputs[0].dtype
                                          : linear_out_dtype(attrs_, x2.dtype, w.dtype);
    TensorDesc o;
    o.rank = 2;
    o.dims[0] = x2.dims[0];
    o.dims[1] = attrs_.gated ? w.dims[0] / 2 : w.dims[0];
    o.dtype = odt;
    return quant_workspace(x2, w, &o, q, odt);
}

Status Linear::compute(std::span<TensorView> outputs, std::span<const TensorView> inputs,
                       const ComputeContext& ctx, void* workspace)
{
    if (Status s = check_views(outputs, inputs); !is_ok(s)) {
        return s;
    }
    if (backend_ != Backend::HIP) {
        return Status::unsupported;
    }
    const TensorDesc descs_in[3] = {inputs[0].desc(), inputs[1].desc(),
                                    inputs.size() > 2 ? inputs[2].desc() : TensorDesc{}};
    const TensorDesc desc_out = outputs[0].desc();
    if (Status s = validate(std::span<const TensorDesc>(descs_in, inputs.size()),
                            std::span<const TensorDesc>(&desc_out, 1));
        !is_ok(s)) {
        return s;
    }
    const TensorView& x = inputs[0];
    const TensorView& wv = inputs[1];
    TensorView& y = outputs[0];
    if (!is_int8_matmul(x.data_type(), wv.data_type()) && !is_q4_1_matmul(x.data_type(), wv.data_type()) &&
        !is_dense_fp_pair(x.data_type(), wv.data_type())) {
        return Status::unsupported;  // nnops' Linear has no fp-activation x s8 route
    }
    if (y.data_type() != linear_out_dtype(attrs_, x.data_type(), wv.data_type()) &&
        !(is_q4_1_matmul(x.data_type(), wv.data_type()) && y.data_type() == DataType::f32)) {
        return Status::invalid_argument;
    }
    // Flatten the leading dims: [..., K] -> [rows, K], [..., N] -> [rows, N].
    const int64_t rows = x.total_rows();
    const int64_t n_out = attrs_.gated ? wv.shape(0) / 2 : wv.shape(0);
    if (y.total_rows() != rows || y.shape(y.rank() - 1) != n_out) {
        return Status::invalid_argument;
    }
    const int64_t xs[2] = {rows, x.shape(x.rank() - 1)};
    const int64_t ys[2] = {rows, n_out};
    const int64_t x_pitch = x.rank() >= 2 ? x.pitch()
                                          : static_cast<int64_t>(data_type_row_bytes(x.data_type(), xs[1]));
    const int64_t y_pitch = y.rank() >= 2 ? y.pitch()
                                          : static_cast<int64_t>(data_type_row_bytes(y.data_type(), ys[1]));
    TensorView x2(xs, x.data_type(), x.ptr<void>(), x_pitch, TensorLayout::Dense, x.quant_params());
    TensorView y2(ys, y.data_type(), y.ptr<void>(), y_pitch, TensorLayout::Dense, y.quant_params());
    TensorView ins[3] = {x2, wv, inputs.size() > 2 ? inputs[2] : TensorView{}};

    const QuantCall q = linear_call(attrs_, inputs.size() > 2);
    const size_t ws = getWorkspaceSize(std::span<const TensorDesc>(descs_in, inputs.size()),
                                       std::span<const TensorDesc>(&desc_out, 1));
    return run_quant(q, y2, std::span<const TensorView>(ins, inputs.size()), ctx, workspace,
                     workspace != nullptr ? ws : 0);
}

// ===========================================================================
// prepackWeights: s8 B, and q4_1 B with blocks along N -> TensorLayout::PackedBHip
// ===========================================================================
namespace {

/// The query / fill contract of nnops' prepackWeights (src/ops/matmul.cpp:
/// 96-141): an empty outputs[0] is the query and receives the descriptor
/// [N, K] (s8, PackedBHip, its row pitch ceil(bytes / N) so that N rows cover
/// the blob, carrying the weight's QuantParams); a populated one is filled on ctx's stream. A
/// weight with no packed form (anything but a 2-D s8 B or a 2-D q4_1 B with
/// blocks along N) answers empty.
Status prepack_q4_1(const TensorView& raw, std::span<TensorView> outputs, const ComputeContext& ctx);

Status prepack_s8(const TensorView& raw, bool trans_b, std::span<TensorView> outputs, const ComputeContext& ctx,
                  Backend backend)
{
    if (outputs.empty()) {
        return Status::invalid_argument;
    }
    if (backend == Backend::HIP && raw.rank() == 2 && raw.data_type() == DataType::q4_1 && !trans_b &&
        raw.layout() == TensorLayout::Dense) {
        return prepack_q4_1(raw, outputs, ctx);
    }
    if (backend != Backend::HIP || raw.rank() != 2 || raw.data_type() != DataType::s8 ||
        raw.layout() != TensorLayout::Dense) {
        if (outputs[0].is_empty()) {
            outputs[0] = TensorView{};
            return Status::ok;
        }
        return Status::unsupported;
    }
    const int64_t n = trans_b ? raw.shape(0) : raw.shape(1);
    const int64_t k = trans_b ? raw.shape(1) : raw.shape(0);
    if (n <= 0 || k <= 0) {
        if (outputs[0].is_empty()) {
            outputs[0] = TensorView{};
            return Status::ok;
        }
        return Status::invalid_argument;
    }
    // described as [N, K] (K exact, so a call can check A against it) with a
    // row pitch large enough for N rows to cover the blob
    const int64_t bytes = static_cast<int64_t>(nnops_hip_prepack_i8_bytes(k, n));
    const int64_t pitch = std::max(k, (bytes + n - 1) / n);
    const int64_t shape[2] = {n, k};
    if (outputs[0].is_empty()) {
        outputs[0] = TensorView(shape, DataType::s8, nullptr, pitch, TensorLayout::PackedBHip, raw.quant_params());
        return Status::ok;
    }
    const TensorView& o = outputs[0];
    if (o.layout() != TensorLayout::PackedBHip || o.data_type() != DataType::s8 || o.rank() != 2 ||
        o.shape(0) != n || o.shape(1) != k || o.pitch() != pitch) {
        return Status::invalid_argument;  // the packed buffer does not match the geometry
    }
    const int rc = nnops_hip_prepack_i8(raw.ptr<const int8_t>(), k, n, raw.row_stride_elems(), trans_b ? 1 : 0,
                                        o.ptr<void>(), ctx.hip_stream);
    return from_code(rc);
}

/// A blocks-along-N q4_1 weight [K, N] (values) -> PackedBHip q4_1 [N, K]:
/// the blob of nnops_hip_prepack_q4_1, with a row pitch whose N rows cover it. Blocks along K (transpose_b) have no packed form.
Status prepack_q4_1(const TensorView& raw, std::span<TensorView> outputs, const ComputeContext& ctx)
{
    const int64_t k = raw.shape(0), n = raw.shape(1);
    if (n <= 0 || k <= 0) {
        if (outputs[0].is_empty()) {
            outputs[0] = TensorView{};
            return Status::ok;
        }
        return Status::invalid_argument;
    }
    // described as [N, K] (K exact) with a row pitch of whole blocks large
    // enough for N rows to cover the two planes
    const int64_t bytes = static_cast<int64_t>(nnops_hip_prepack_q4_1_bytes(k, n));
    const int64_t pitch = 20 * std::max((k + 31) / 32, (bytes + n * 20 - 1) / (n * 20));
    const int64_t shape[2] = {n, k};
    if (outputs[0].is_empty()) {
        outputs[0] = TensorView(shape, DataType::q4_1, nullptr, pitch, TensorLayout::PackedBHip, raw.quant_params());
        return Status::ok;
    }
    const TensorView& o = outputs[0];
    if (o.layout() != TensorLayout::PackedBHip || o.data_type() != DataType::q4_1 || o.rank() != 2 ||
        o.shape(0) != n || o.shape(1) != k || o.pitch() != pitch) {
        return Status::invalid_argument;
    }
    const int rc = nnops_hip_prepack_q4_1(raw.ptr<const uint8_t>(), k, n, raw.pitch(), 0, o.ptr<void>(),
                                          ctx.hip_stream);
    return from_code(rc);
}

}  // namespace

Status MatMul::prepack(std::span<const TensorView> inputs, std::span<TensorView> outputs, const ComputeContext& ctx)
{
    if (inputs.empty()) {
        return Status::invalid_argument;
    }
    return prepack_s8(inputs[0], attrs_.transpose_b, outputs, ctx, backend_);
}

void MatMul::prepackWeights(std::span<const TensorView> inputs, std::span<TensorView> outputs,
                            const ComputeContext& ctx)
{
    (void)prepack(inputs, outputs, ctx);
}

Status Linear::prepack(std::span<const TensorView> inputs, std::span<TensorView> outputs, const ComputeContext& ctx)
{
    if (inputs.empty()) {
        return Status::invalid_argument;
    }
    return prepack_s8(inputs[0], true, outputs, ctx, backend_);  // the weight is [N, K]
}

void Linear::prepackWeights(std::span<const TensorView> inputs, std::span<TensorView> outputs,
                            const ComputeContext& ctx)
{
    (void)prepack(inputs, outputs, ctx);
}

}  // namespace nnops
