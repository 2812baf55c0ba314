// Device-side building blocks shared by the gfx950 kernels: vector types, the
// int8 output pass (compensate -> bias -> Relu -> requant) and the float
// epilogue, written so every float operation rounds on its own (these TUs are
// compiled with -ffp-contract=off), which is what makes integer outputs
// bit-identical to nnops' scalar requant.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "nnops_amd.h"

namespace nnops_amd {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Wait until at most N vector-memory operations of this wave are outstanding
// (they retire in issue order, global_load_lds included).
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// The calling thread's armed kernel-timing events (nnops_hip_time_next_launch):
// the next launch through NNOPS_LAUNCH carries them on its dispatch packet
// (hipExtLaunchKernelGGL) and disarms them.
struct LaunchTiming {
    hipEvent_t start = nullptr, stop = nullptr;
};
inline LaunchTiming& launch_timing()
{
    static thread_local LaunchTiming t;
    return t;
}

template <typename F, typename... Args>
inline void nnops_launch(F kernel, const dim3& grid, const dim3& block, uint32_t shmem, hipStream_t stream,
                         Args... args)
{
    LaunchTiming& t = launch_timing();
    if (t.start != nullptr) {
        const LaunchTiming armed = t;
        t = LaunchTiming{};
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, armed.start, armed.stop, 0u, args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, shmem, stream, args...);
    }
}
#define NNOPS_LAUNCH(kernel, ...) ::nnops_amd::nnops_launch(kernel, __VA_ARGS__)

// Disarms the calling thread's timing events when a public entry point
// returns, so a call that returns before launching (a rejected argument, an
// empty problem) leaves no armed pair for an unrelated later kernel.
struct TimingDisarm {
    TimingDisarm() = default;
    TimingDisarm(const TimingDisarm&) = delete;
    TimingDisarm& operator=(const TimingDisarm&) = delete;
    ~TimingDisarm() { launch_timing() = LaunchTiming{}; }
};

// Launch epochs for the split-completion flags of the one-launch split
// kernels: unique in the process and never 0. Consecutive counter values are
// spread over 64 bits (splitmix64's finalizer), so a flag word that a caller's
// workspace happens to hold from other work (small integers, float partials)
// does not pass for this launch's epoch.
inline uint64_t next_launch_epoch()
{
    static std::atomic<uint64_t> counter{0};
    uint64_t z = counter.fetch_add(1, std::memory_order_relaxed) + 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    return z != 0 ? z : 1;
}

// ---------------------------------------------------------------------------
// Epilogue parameters, resolved once on the host (device pointers only).
// ---------------------------------------------------------------------------
struct EpiParams {
    const int32_t* bias;       // [N] int32 (integer outputs) or nullptr
    const int32_t* r_a;        // [M] sum_k A (true values), or nullptr
    const int32_t* r_b;        // [N] sum_k B, or nullptr
    const float* s_a;          // [M] or nullptr -> s_a_scalar
    const int32_t* zp_a;       // [M] or nullptr -> zp_a_scalar
    const float* s_b;          // [N] or nullptr -> s_b_scalar
    const int32_t* zp_b;       // [N] or nullptr -> zp_b_scalar
    const float* s_out_rows;   // [M] or nullptr -> s_out
    const int32_t* zp_out_rows;
    float s_a_scalar, s_b_scalar, s_out;
    int32_t zp_a_scalar, zp_b_scalar, zp_out;
    int32_t a_off;             // shift left in the accumulate: -128 for a u8 A read as s8
    int32_t k;
    int32_t out_kind;          // NNOPS_OUT_*
    int32_t act;               // NNOPS_ACT_*
    int32_t round_even;
    int32_t float_ep;
    float min_clip, max_clip;
    int32_t add_to, residual_pre;
    int32_t compensate;        // any of r_a / r_b is live
    const void* bias_fp;       // [N] bias in the f32/f16 destination's type, or nullptr
    float act_alpha, act_beta; // LeakyRelu / Elu alpha, HardSwish beta
};

__host__ __device__ __forceinline__ bool epi_is_fp(const EpiParams& p)
{
    return p.out_kind == NNOPS_OUT_F32 || p.out_kind == NNOPS_OUT_F16;
}

// a / b for a divisor b fixed over many divisions, given y = RN(1/b): one
// Markstein correction of the reciprocal product (q0 = RN(a y), r = a - b q0
// exactly by the fma, q = RN(q0 + r y)). By Markstein's theorem (IBM J. Res.
// Dev. 34(1), 1990) q is the correctly rounded a / b, the same bits as
// __fdiv_rn, barring overflow and underflow, which the output passes' operands
// (bounded integer accumulators times positive scales) do not reach; five
// instructions in place of the division's eleven.
__device__ __forceinline__ float div_by_fixed(float a, float b, float y)
{
    const float q0 = __fmul_rn(a, y);
    const float r = __builtin_fmaf(-q0, b, a);
    return __builtin_fmaf(r, y, q0);
}

// Per-row constants of the output pass.
struct EpiRow {
    int32_t zp_a, r_a, zp_out;
    float s_a, s_out, row_k, inv_out;
};

__device__ __forceinline__ EpiRow epi_row(const EpiParams& p, int m)
{
    EpiRow r;
    r.zp_a = p.zp_a ? p.zp_a[m] : p.zp_a_scalar;
    r.r_a = p.r_a ? p.r_a[m] : 0;
    r.s_a = p.s_a ? p.s_a[m] : p.s_a_scalar;
    r.s_out = p.s_out_rows ? p.s_out_rows[m] : p.s_out;
    r.zp_out = p.zp_out_rows ? p.zp_out_rows[m] : p.zp_out;
    r.row_k = __fdiv_rn(r.s_a, r.s_out);
    r.inv_out = __fdiv_rn(1.0f, r.s_out);
    return r;
}

// Per-column constants of the output pass.
struct EpiCol {
    int32_t bias, zp_b, r_b;
    float s_b;
};

__device__ __forceinline__ EpiCol epi_col(const EpiParams& p, int n)
{
    EpiCol c;
    c.bias = p.bias ? p.bias[n] : 0;
    c.zp_b = p.zp_b ? p.zp_b[n] : p.zp_b_scalar;
    c.r_b = p.r_b ? p.r_b[n] : 0;
    c.s_b = p.s_b ? p.s_b[n] : p.s_b_scalar;
    return c;
}

// Recover sum_k (a - zp_a)(b - zp_b) from the raw accumulate: the same algebra
// as nnops' matmul_int8_compensate, with a_off the shift the kernel left in.
__device__ __forceinline__ int32_t epi_compensate(const EpiParams& p, const EpiRow& r,
                                                  const EpiCol& c, int32_t raw)
{
    if (!p.compensate) {
        return raw;
    }
    return raw - (p.a_off + r.zp_a) * c.r_b - c.zp_b * r.r_a + p.k * r.zp_a * c.zp_b;
}

__device__ __forceinline__ float round_half_away(float x)
{
    return __builtin_truncf(__fadd_rn(x, __builtin_copysignf(0.5f, x)));
}

__device__ __forceinline__ int32_t requant_clamped(float x, int32_t zp, bool u8, bool even)
{
    const float zpf = (float)zp;
    const float lo = __fsub_rn(u8 ? 0.0f : -128.0f, zpf);
    const float hi = __fsub_rn(u8 ? 255.0f : 127.0f, zpf);
    // clamp to [lo, hi] (lo < hi) in one v_med3_f32: the same value as the
    // two compares for every number x (the int8 passes never hand it a NaN)
    x = __builtin_amdgcn_fmed3f(x, lo, hi);
    const float rr = even ? __builtin_rintf(x) : round_half_away(x);
    return (int32_t)rr + zp;
}

// tanh(|x|) = (1 - t)/(1 + t), t = exp(-2|x|), exp by Cody & Waite's reduction
// (Software Manual for the Elementary Functions, 1980) and the degree-7 Taylor
// polynomial of exp(-r) on |r| <= ln2/2 in Horner form. Built only from
// correctly rounded +,-,*,/ and floor, so the host evaluates the same bits.
__device__ __forceinline__ float tanh_cw(float x)
{
    // |x| >= 9 (and NaN) is selected at the end rather than branched to: the
    // reduction runs on min(|x|, 9), the same operations for every |x| < 9
    const float ax0 = __builtin_fabsf(x);
    const bool big = !(ax0 < 9.0f);
    const float ax = big ? 9.0f : ax0;
    const float y = __fadd_rn(ax, ax);
    const float n = __builtin_floorf(__fadd_rn(__fmul_rn(y, 1.44269504088896341f), 0.5f));
    const float r = __fsub_rn(__fsub_rn(y, __fmul_rn(n, 0.693145751953125f)),
                              __fmul_rn(n, 1.42860682030941723e-06f));
    const float nr = -r;
    float q = 1.98412698412698413e-04f;
    q = __fadd_rn(__fmul_rn(q, nr), 1.38888888888888889e-03f);
    q = __fadd_rn(__fmul_rn(q, nr), 8.33333333333333333e-03f);
    q = __fadd_rn(__fmul_rn(q, nr), 4.16666666666666667e-02f);
    q = __fadd_rn(__fmul_rn(q, nr), 1.66666666666666667e-01f);
    q = __fadd_rn(__fmul_rn(q, nr), 0.5f);
    q = __fadd_rn(__fmul_rn(q, nr), 1.0f);
    q = __fadd_rn(__fmul_rn(q, nr), 1.0f);
    const int ni = (int)n;
    const float scale = __int_as_float((127 - ni) << 23);
    const float t = __fmul_rn(q, scale);
    const float th = __fdiv_rn(__fsub_rn(1.0f, t), __fadd_rn(1.0f, t));
    return big ? ((x != x) ? x : __builtin_copysignf(1.0f, x)) : __builtin_copysignf(th, x);
}

// GELU, tanh form, in nnops' operation order: 0.5x(1 + tanh(c(x + 0.044715x^3))).
__device__ __forceinline__ float gelu_tanh(float x)
{
    const float c = 0.7978845608028654f;
    const float x3 = __fmul_rn(__fmul_rn(__fmul_rn(0.044715f, x), x), x);
    const float inner = __fmul_rn(c, __fadd_rn(x, x3));
    return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, tanh_cw(inner)));
}

__device__ __forceinline__ float apply_act(const EpiParams& p, float x)
{
    x = x < p.min_clip ? p.min_clip : x;
    x = p.max_clip < x ? p.max_clip : x;
    if (p.act == NNOPS_ACT_RELU) {
        return x > 0.0f ? x : 0.0f;
    }
    if (p.act == NNOPS_ACT_GELU) {
        return gelu_tanh(x);
    }
    return x;
}

// nnops' activation set on the dequantized value, after the clip
// (apply_epilogue, simd_epilogue.hpp:56-90); exp and tanh are the device
// library's.
__device__ __forceinline__ float apply_act_fp(const EpiParams& p, float x)
{
    x = x < p.min_clip ? p.min_clip : x;
    x = p.max_clip < x ? p.max_clip : x;
    switch (p.act) {
    case NNOPS_ACT_RELU:
        return x > 0.0f ? x : 0.0f;
    case NNOPS_ACT_RELU6: {
        const float y = x > 0.0f ? x : 0.0f;
        return y < 6.0f ? y : 6.0f;
    }
    case NNOPS_ACT_LEAKY_RELU:
        return x > 0.0f ? x : __fmul_rn(p.act_alpha, x);
    case NNOPS_ACT_SIGMOID:
        return __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-x)));
    case NNOPS_ACT_TANH:
        return tanhf(x);
    case NNOPS_ACT_GELU: {
        const float c = 0.7978845608028654f;
        const float x3 = __fmul_rn(__fmul_rn(__fmul_rn(0.044715f, x), x), x);
        return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, tanhf(__fmul_rn(c, __fadd_rn(x, x3)))));
    }
    case NNOPS_ACT_SILU:
        return __fdiv_rn(x, __fadd_rn(1.0f, expf(-x)));
    case NNOPS_ACT_HARDSWISH: {
        float r6 = __fadd_rn(x, 3.0f);
        r6 = r6 > 0.0f ? r6 : 0.0f;
        r6 = r6 < 6.0f ? r6 : 6.0f;
        return __fmul_rn(__fmul_rn(x, r6), __fdiv_rn(p.act_beta, 6.0f));
    }
    case NNOPS_ACT_ELU:
        return x > 0.0f ? x : __fmul_rn(p.act_alpha, __fsub_rn(expf(x), 1.0f));
    default:
        return x;
    }
}

// The dequantizing output pass (nnops' DqRoute, dq_epilogue_row,
// simd_epilogue.hpp:784-949, and tests/reference/matmul_dq_ref.cpp:178-190):
// f = float(v) * (s_a * s_b) [+ bias[n]], then the residual, clip and activation.
__device__ __forceinline__ float epi_value_fp(const EpiParams& p, const EpiRow& r, int n, int32_t raw,
                                              float old)
{
    const EpiCol col = epi_col(p, n);
    const int32_t v = epi_compensate(p, r, col, raw);
    float f = __fmul_rn((float)v, __fmul_rn(r.s_a, col.s_b));
    if (p.bias_fp != nullptr) {
        const float b = p.out_kind == NNOPS_OUT_F16 ? (float)static_cast<const _Float16*>(p.bias_fp)[n]
                                                    : static_cast<const float*>(p.bias_fp)[n];
        f = __fadd_rn(f, b);
    }
    // a pre-activation residual joins before the clip; a post-activation one
    // is added to the destination-typed result (nnops' Linear: a compact
    // temporary, then residual_add, src/backend/cpu/matmul/linear.cpp:283-301)
    if (p.add_to && p.residual_pre) {
        f = __fadd_rn(f, old);
    }
    f = apply_act_fp(p, f);
    if (p.add_to && !p.residual_pre) {
        if (p.out_kind == NNOPS_OUT_F16) {
            f = (float)(_Float16)f;
        }
        f = __fadd_rn(f, old);
    }
    return f;
}

// The output pass for one element: raw int32 accumulate in, the value to store
// out (int32 for s32, the s8/u8 code otherwise). `old` is the destination's
// current value, read only when add_to.
__device__ __forceinline__ int32_t epi_value(const EpiParams& p, const EpiRow& r, const EpiCol& col,
                                             int32_t raw, int32_t old)
{
    int32_t v = epi_compensate(p, r, col, raw) + col.bias;
    if (p.out_kind == NNOPS_OUT_S32) {
        return (p.act == NNOPS_ACT_RELU && v < 0) ? 0 : v;
    }
    const bool u8 = p.out_kind == NNOPS_OUT_U8;
    if (!p.float_ep) {
        if (p.act == NNOPS_ACT_RELU) {
            v = v < 0 ? 0 : v;
        }
        const float req = __fmul_rn(r.row_k, col.s_b);
        return requant_clamped(__fmul_rn((float)v, req), r.zp_out, u8, p.round_even);
    }
    float f = __fmul_rn((float)v, __fmul_rn(r.s_a, col.s_b));
    float res = 0.0f;
    if (p.add_to) {
        res = __fmul_rn((float)(old - r.zp_out), r.s_out);
        if (p.residual_pre) {
            f = __fadd_rn(f, res);
        }
    }
    f = apply_act(p, f);
    if (p.add_to && !p.residual_pre) {
        f = __fadd_rn(f, res);
    }
    return requant_clamped(div_by_fixed(f, r.s_out, r.inv_out), r.zp_out, u8, p.round_even);
}

__device__ __forceinline__ int32_t epi_load_old(const EpiParams& p, const void* crow, int n)
{
    if (!p.add_to) {
        return 0;
    }
    return p.out_kind == NNOPS_OUT_U8 ? (int32_t) static_cast<const uint8_t*>(crow)[n]
                                      : (int32_t) static_cast<const int8_t*>(crow)[n];
}

// Single-element store of the output pass.
__device__ __forceinline__ void epi_store(const EpiParams& p, const EpiRow& r, const EpiCol& col,
                                          int32_t raw, void* crow, int n)
{
    if (p.out_kind == NNOPS_OUT_F32) {
        float* c = static_cast<float*>(crow) + n;
        *c = epi_value_fp(p, r, n, raw, p.add_to ? *c : 0.0f);
        return;
    }
    if (p.out_kind == NNOPS_OUT_F16) {
        _Float16* c = static_cast<_Float16*>(crow) + n;
        *c = (_Float16)epi_value_fp(p, r, n, raw, p.add_to ? (float)*c : 0.0f);
        return;
    }
    const int32_t q = epi_value(p, r, col, raw, epi_load_old(p, crow, n));
    if (p.out_kind == NNOPS_OUT_S32) {
        static_cast<int32_t*>(crow)[n] = q;
    } else {
        static_cast<int8_t*>(crow)[n] = (int8_t)q;
    }
}

// Bytes of the destination element for an out kind.
__host__ __device__ __forceinline__ int out_elem_bytes(int out_kind)
{
    return (out_kind == NNOPS_OUT_S32 || out_kind == NNOPS_OUT_F32) ? 4
           : (out_kind == NNOPS_OUT_F16) ? 2 : 1;
}

}  // namespace nnops_amd
