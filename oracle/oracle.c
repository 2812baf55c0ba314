/* CPU oracle for the quantized-matmul path. Test infrastructure only: see
 * oracle.h for who may load it and how each function is pinned.
 *
 * Reference citations are paths in the nnops source tree.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static inline float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* ---------------------------------------------------------------------------
 * f16 <-> f32 (include/nnops/detail/half.hpp:69-134 semantics: exact widening,
 * round-to-nearest-even narrowing, overflow to infinity, NaN -> quiet NaN).
 * Written from the IEEE 754 binary16 definition.
 * ------------------------------------------------------------------------- */
float orc_f16_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t mant = h & 0x3ffu;
    if (e == 0x1fu) {
        return bits_to_f32(sign | 0x7f800000u | (mant << 13));
    }
    if (e == 0) {
        /* zero or subnormal: mant * 2^-24, exact in f32 */
        const float v = (float)mant * (1.0f / 16777216.0f);
        return bits_to_f32(sign | f32_to_bits(v));
    }
    return bits_to_f32(sign | ((e + 112u) << 23) | (mant << 13));
}

uint16_t orc_f32_to_f16(float f)
{
    const uint32_t x = f32_to_bits(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) {
        return (uint16_t)(sign | 0x7e00u);
    }
    if (ax >= 0x477ff000u) { /* >= 65520 rounds to infinity */
        return (uint16_t)(sign | 0x7c00u);
    }
    const int32_t e = (int32_t)(ax >> 23);
    if (ax < 0x38800000u) { /* below 2^-14: half subnormal or zero */
        if (e == 0) {
            return sign; /* f32 subnormals are far below half's smallest step */
        }
        const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
        const int32_t s = 126 - e; /* value = mant * 2^(e-150) = (mant >> s) units of 2^-24 */
        if (s > 24) {
            return sign;
        }
        uint32_t q = mant >> s;
        const uint32_t rem = mant & ((1u << s) - 1u);
        const uint32_t half = 1u << (s - 1);
        if (rem > half || (rem == half && (q & 1u))) {
            ++q;
        }
        return (uint16_t)(sign | q);
    }
    const uint32_t mant = ax & 0x7fffffu;
    uint32_t q = ((uint32_t)(e - 112) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) {
        ++q;
    }
    return (uint16_t)(sign | q);
}

/* ---------------------------------------------------------------------------
 * Integer GEMM. Follows tests/reference/matmul_int8_ref.cpp:36-217:
 * raw = sum_k a*b over the operands' own element types, compensated as
 * simd_epilogue.hpp:129-133, + int32 bias, Relu, then requant
 * (simd_epilogue.hpp:137-160); the output scale is the destination's per-tensor
 * one unless a per-row table is given (matmul_tile_impl.h:399-410).
 * ------------------------------------------------------------------------- */
float orc_requant_scale(float s_a, float s_b, float s_out)
{
    /* (s_a / s_out) * s_b, simd_epilogue.hpp:157-160 */
    const float row_k = s_a / s_out;
    return row_k * s_b;
}

static float round_half_away(float x)
{
    /* std::trunc(x + copysign(0.5, x)) in f32, simd_epilogue.hpp:145 */
    const float h = copysignf(0.5f, x);
    const float y = x + h;
    return truncf(y);
}

int32_t orc_requant(int32_t acc, float req, int32_t zp, int32_t u8, int32_t round_even)
{
    const float kmin = u8 ? 0.0f : -128.0f;
    const float kmax = u8 ? 255.0f : 127.0f;
    const float zpf = (float)zp;
    float x = (float)acc * req;
    const float lo = kmin - zpf;
    const float hi = kmax - zpf;
    if (x < lo) x = lo;
    if (hi < x) x = hi;
    const float r = round_even ? rintf(x) : round_half_away(x);
    return (int32_t)r + zp;
}

/* Float requant used by the float epilogue: q = clamp(round(y / s_out)) + zp. */
static int32_t requant_float(float y, float s_out, int32_t zp, int32_t u8, int32_t round_even)
{
    const float kmin = u8 ? 0.0f : -128.0f;
    const float kmax = u8 ? 255.0f : 127.0f;
    const float zpf = (float)zp;
    float x = y / s_out;
    const float lo = kmin - zpf;
    const float hi = kmax - zpf;
    if (x < lo) x = lo;
    if (hi < x) x = hi;
    const float r = round_even ? rintf(x) : round_half_away(x);
    return (int32_t)r + zp;
}

/* tanh for the GELU epilogue: tanh(|x|) = (1 - t) / (1 + t), t = exp(-2|x|),
 * with exp by Cody & Waite's argument reduction (Software Manual for the
 * Elementary Functions, 1980): n = round(y / ln2), r = y - n*ln2 split in a
 * hi/lo pair, exp(-r) by its degree-7 Taylor polynomial in Horner form, then
 * an exact power-of-two scale. Absolute error ~1e-7, which is what GELU's
 * 1 + tanh needs. Only +,-,*,/ and floor are used, so the HIP kernels evaluate
 * the same float operations to the same bits. */
float orc_tanhf(float x)
{
    const float ax = fabsf(x);
    if (!(ax < 9.0f)) {
        return (x != x) ? x : copysignf(1.0f, x);
    }
    const float y = ax + ax;                          /* exp(-y), y in [0, 18) */
    const float n = floorf(y * 1.44269504088896341f + 0.5f);
    const float r = (y - n * 0.693145751953125f) - n * 1.42860682030941723e-06f;
    /* exp(-r), |r| <= ln2/2 */
    const float nr = -r;
    float p = 1.98412698412698413e-04f;               /* 1/5040 */
    p = p * nr + 1.38888888888888889e-03f;             /* 1/720 */
    p = p * nr + 8.33333333333333333e-03f;             /* 1/120 */
    p = p * nr + 4.16666666666666667e-02f;             /* 1/24 */
    p = p * nr + 1.66666666666666667e-01f;             /* 1/6 */
    p = p * nr + 0.5f;
    p = p * nr + 1.0f;
    p = p * nr + 1.0f;
    const int32_t ni = (int32_t)n;                     /* 0..26 */
    const float scale = bits_to_f32((uint32_t)(127 - ni) << 23);
    const float t = p * scale;
    const float th = (1.0f - t) / (1.0f + t);
    return copysignf(th, x);
}

/* Division by a fixed divisor as the HIP output passes evaluate it:
 * y = RN(1/b) once, q0 = RN(a*y), r = fma(-q0, b, a) (exact), q = fma(r, y, q0).
 * Markstein's theorem (IBM J. Res. Dev. 34(1), 1990: with y the correctly
 * rounded reciprocal and q0 within an ulp of a/b, one such correction gives
 * the correctly rounded quotient) says q = RN(a/b) barring overflow and
 * underflow. Counts the a in [lo, hi) (float bit patterns, every `step`-th)
 * where the sequence and IEEE division differ: the tests check that it is 0
 * (corrected = 0 stops at q0, the plain reciprocal multiply, which differs). */
int64_t orc_markstein_mismatches(float b, uint32_t lo, uint32_t hi, uint32_t step, int32_t corrected)
{
    volatile float one = 1.0f;
    const float y = one / b;
    int64_t bad = 0;
    for (uint64_t u = lo; u < hi; u += step) {
        const float a = bits_to_f32((uint32_t)u);
        const float q0 = a * y;
        const float r = fmaf(-q0, b, a);
        const float q = corrected ? fmaf(r, y, q0) : q0;
        if (f32_to_bits(q) != f32_to_bits(a / b)) {
            ++bad;
        }
    }
    return bad;
}

/* GELU, tanh approximation, with the reference's operation order
 * (simd_epilogue.hpp:76-79). */
float orc_gelu_tanh(float x)
{
    const float c = 0.7978845608028654f;
    const float x3 = ((0.044715f * x) * x) * x;
    const float inner = c * (x + x3);
    return (0.5f * x) * (1.0f + orc_tanhf(inner));
}

static float apply_act_ab(int32_t act, float x, float lo, float hi, float alpha, float beta)
{
    /* apply_epilogue: activate(clamp(x, min_clip, max_clip)), simd_epilogue.hpp:56-90 */
    if (x < lo) x = lo;
    if (hi < x) x = hi;
    switch (act) {
    case ORC_ACT_RELU: return x > 0.0f ? x : 0.0f;
    case ORC_ACT_RELU6: { float y = x > 0.0f ? x : 0.0f; return y < 6.0f ? y : 6.0f; }
    case ORC_ACT_LEAKY_RELU: return x > 0.0f ? x : alpha * x;
    case ORC_ACT_SIGMOID: return 1.0f / (1.0f + expf(-x));
    case ORC_ACT_TANH: return tanhf(x);
    case ORC_ACT_GELU: return orc_gelu_tanh(x);
    case ORC_ACT_SILU: return x / (1.0f + expf(-x));
    case ORC_ACT_HARDSWISH: {
        float r6 = x + 3.0f;
        r6 = r6 > 0.0f ? r6 : 0.0f;
        r6 = r6 < 6.0f ? r6 : 6.0f;
        return x * r6 * (beta / 6.0f);
    }
    case ORC_ACT_ELU: return x > 0.0f ? x : alpha * (expf(x) - 1.0f);
    default: return x;
    }
}

/* the reference's GELU for dequantized (f32/f16) destinations: std::tanh */
static float apply_act_fp(int32_t act, float x, float lo, float hi, float alpha, float beta)
{
    if (act == ORC_ACT_GELU) {
        if (x < lo) x = lo;
        if (hi < x) x = hi;
        const float c = 0.7978845608028654f;
        return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
    }
    return apply_act_ab(act, x, lo, hi, alpha, beta);
}

static float apply_act(int32_t act, float x, float lo, float hi)
{
    return apply_act_ab(act, x, lo, hi, 0.0f, 1.0f);
}

static inline int32_t load_a(const orc_gemm_i8_t* p, int64_t m, int64_t k)
{
    const int64_t off = p->trans_a ? k * p->lda + m : m * p->lda + k;
    return p->a_u8 ? (int32_t)((const uint8_t*)p->a)[off] : (int32_t)((const int8_t*)p->a)[off];
}

static inline int32_t load_b(const orc_gemm_i8_t* p, int64_t k, int64_t n)
{
    const int64_t off = p->trans_b ? n * p->ldb + k : k * p->ldb + n;
    return (int32_t)p->b[off];
}

void orc_gemm_i8(const orc_gemm_i8_t* p)
{
    const int64_t M = p->m, N = p->n, K = p->k;
    const int64_t m0 = p->m_begin;
    const int64_t m1 = (p->m_end > 0) ? p->m_end : M;
    const int32_t kk = (int32_t)K;

    int32_t* r_b = (int32_t*)calloc((size_t)(N > 0 ? N : 1), sizeof(int32_t));
    int32_t* raw = (int32_t*)calloc((size_t)(N > 0 ? N : 1), sizeof(int32_t));
    for (int64_t n = 0; n < N; ++n) {
        int32_t s = 0;
        for (int64_t k = 0; k < K; ++k) s += load_b(p, k, n);
        r_b[n] = s;
    }

    for (int64_t m = m0; m < m1; ++m) {
        int32_t r_a = 0;
        for (int64_t k = 0; k < K; ++k) r_a += load_a(p, m, k);
        /* raw int32 dot products of row m */
        if (p->trans_b) {
            for (int64_t n = 0; n < N; ++n) {
                int32_t s = 0;
                for (int64_t k = 0; k < K; ++k) s += load_a(p, m, k) * load_b(p, k, n);
                raw[n] = s;
            }
        } else {
            memset(raw, 0, (size_t)N * sizeof(int32_t));
            for (int64_t k = 0; k < K; ++k) {
                const int32_t av = load_a(p, m, k);
                const int8_t* brow = p->b + k * p->ldb;
                for (int64_t n = 0; n < N; ++n) raw[n] += av * (int32_t)brow[n];
            }
        }

        const int32_t zp_a = p->zp_a ? p->zp_a[m] : p->zp_a_scalar;
        const float s_a = p->s_a ? p->s_a[m] : p->s_a_scalar;
        const float s_out = p->s_out_rows ? p->s_out_rows[m] : p->s_out;
        const int32_t zp_out = p->zp_out_rows ? p->zp_out_rows[m] : p->zp_out;

        for (int64_t n = 0; n < N; ++n) {
            const int32_t zp_b = p->zp_b ? p->zp_b[n] : p->zp_b_scalar;
            const float s_b = p->s_b ? p->s_b[n] : p->s_b_scalar;
            /* matmul_int8_compensate with u8_offset 0: the dot was over true values */
            int32_t v = raw[n] - zp_a * r_b[n] - zp_b * r_a + kk * zp_a * zp_b;

            if (p->out_kind == ORC_OUT_F32 || p->out_kind == ORC_OUT_F16) {
                /* dq route (simd_epilogue.hpp:784-949, matmul_dq_ref.cpp:178-190):
                 * f = float(v) * (s_a * s_b) [+ bias[n]]; a pre-activation
                 * residual joins before the clip; a post-activation one is
                 * added to the destination-typed result (linear.cpp:283-301:
                 * a compact temporary, then residual_add). */
                const int f16 = p->out_kind == ORC_OUT_F16;
                float* c32 = (float*)p->c + m * p->ldc + n;
                uint16_t* c16 = (uint16_t*)p->c + m * p->ldc + n;
                const float old = p->add_to ? (f16 ? orc_f16_to_f32(*c16) : *c32) : 0.0f;
                float f = (float)v * (s_a * s_b);
                if (p->bias) {
                    f += f16 ? orc_f16_to_f32(((const uint16_t*)p->bias)[n]) : ((const float*)p->bias)[n];
                }
                if (p->add_to && p->residual_pre) f += old;
                f = apply_act_fp(p->act, f, p->min_clip, p->max_clip, p->act_alpha, p->act_beta);
                if (p->add_to && !p->residual_pre) {
                    if (f16) f = orc_f16_to_f32(orc_f32_to_f16(f));
                    f = f + old;
                }
                if (f16) *c16 = orc_f32_to_f16(f); else *c32 = f;
                continue;
            }

            if (p->bias) v += ((const int32_t*)p->bias)[n];

            if (p->out_kind == ORC_OUT_S32) {
                if (p->act == ORC_ACT_RELU && v < 0) v = 0;
                ((int32_t*)p->c)[m * p->ldc + n] = v;
                continue;
            }

            const int32_t u8 = (p->out_kind == ORC_OUT_U8);
            int32_t q;
            if (!p->float_ep) {
                if (p->act == ORC_ACT_RELU && v < 0) v = 0;
                q = orc_requant(v, orc_requant_scale(s_a, s_b, s_out), zp_out, u8, p->round_even);
            } else {
                /* Float epilogue on an integer destination (no reference route):
                 *   f = float(acc) * (s_a * s_b)                 dq order
                 *   r = float(c_old - zp_out) * s_out           residual, real units
                 *   y = act(clip(f [+ r if pre])) [+ r if post]
                 *   q = clamp(round(y / s_out)) + zp_out
                 */
                float f = (float)v * (s_a * s_b);
                float r = 0.0f;
                if (p->add_to) {
                    const int32_t old = u8 ? (int32_t)((uint8_t*)p->c)[m * p->ldc + n]
                                           : (int32_t)((int8_t*)p->c)[m * p->ldc + n];
                    r = (float)(old - zp_out) * s_out;
                }
                if (p->add_to && p->residual_pre) f += r;
                f = apply_act(p->act, f, p->min_clip, p->max_clip);
                if (p->add_to && !p->residual_pre) f += r;
                q = requant_float(f, s_out, zp_out, u8, p->round_even);
            }
            if (u8) {
                ((uint8_t*)p->c)[m * p->ldc + n] = (uint8_t)q;
            } else {
                ((int8_t*)p->c)[m * p->ldc + n] = (int8_t)q;
            }
        }
    }
    free(r_b);
    free(raw);
}

/* ---------------------------------------------------------------------------
 * Q4_1 codec: include/nnops/detail/q4_1.hpp:62-79 (decode: y = d*q + m in f32,
 * low nibble of byte j -> value j, high nibble -> value j+16) and :92-149
 * (llama.cpp quantize_row_q4_1_ref: d = (max-min)/15, m = min, q = trunc((x -
 * min) * (1/d) + 0.5) clamped to 15).
 * ------------------------------------------------------------------------- */
static void decode_block(const uint8_t* blk, float* out)
{
    uint16_t db, mb;
    memcpy(&db, blk, 2);
    memcpy(&mb, blk + 2, 2);
    const float d = orc_f16_to_f32(db);
    const float m = orc_f16_to_f32(mb);
    for (int j = 0; j < 16; ++j) {
        const float lo = (float)(blk[4 + j] & 0x0f);
        const float hi = (float)(blk[4 + j] >> 4);
        const float pl = d * lo;
        const float ph = d * hi;
        out[j] = pl + m;
        out[j + 16] = ph + m;
    }
}

void orc_q4_1_decode(const void* blocks, int64_t count, float* out)
{
    const uint8_t* src = (const uint8_t*)blocks;
    float tmp[32];
    for (int64_t base = 0; base < count; base += 32) {
        decode_block(src + (base / 32) * 20, tmp);
        const int64_t n = (count - base) < 32 ? (count - base) : 32;
        for (int64_t j = 0; j < n; ++j) out[base + j] = tmp[j];
    }
}

void orc_q4_1_quantize(const float* src, int64_t count, void* blocks)
{
    uint8_t* dst = (uint8_t*)blocks;
    for (int64_t base = 0, b = 0; base < count; base += 32, ++b) {
        const int n = (int)((count - base) < 32 ? (count - base) : 32);
        const float* x = src + base;
        float vmin = x[0], vmax = x[0];
        for (int j = 1; j < n; ++j) {
            vmin = x[j] < vmin ? x[j] : vmin;
            vmax = x[j] > vmax ? x[j] : vmax;
        }
        const float d = (vmax - vmin) / 15.0f;
        const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
        uint8_t* blk = dst + b * 20;
        const uint16_t dh = orc_f32_to_f16(d);
        const uint16_t mh = orc_f32_to_f16(vmin);
        memcpy(blk, &dh, 2);
        memcpy(blk + 2, &mh, 2);
        uint8_t qs[16];
        memset(qs, 0, sizeof(qs));
        for (int j = 0; j < n; ++j) {
            const float qf = (x[j] - vmin) * id + 0.5f;
            const uint8_t q = (uint8_t)(qf < 15.0f ? (int)qf : 15);
            if (j < 16) qs[j] = q;
            else qs[j - 16] |= (uint8_t)(q << 4);
        }
        memcpy(blk + 4, qs, 16);
    }
}

/* ---------------------------------------------------------------------------
 * f32 dequant GEMM over Q4_1 weights: tests/test_matmul_q4_1.cpp:190-224
 * (decode the weights in f32, upcast A exactly, accumulate; with an f16 A the
 * decoded weight is rounded to f16 and the output rounds once at the store).
 * ------------------------------------------------------------------------- */
void orc_gemm_q4_1(const orc_gemm_q4_1_t* p)
{
    const int64_t M = p->m, N = p->n, K = p->k;
    const int64_t m0 = p->m_begin;
    const int64_t m1 = (p->m_end > 0) ? p->m_end : M;
    /* dense decoded W^T: [N][K] floats */
    float* w = (float*)malloc((size_t)(N * K > 0 ? N * K : 1) * sizeof(float));
    float* a = (float*)malloc((size_t)(K > 0 ? K : 1) * sizeof(float));
    if (p->trans_b) {
        for (int64_t n = 0; n < N; ++n) orc_q4_1_decode(p->b + n * p->ldb_bytes, K, w + n * K);
    } else {
        float* row = (float*)malloc((size_t)(N > 0 ? N : 1) * sizeof(float));
        for (int64_t k = 0; k < K; ++k) {
            orc_q4_1_decode(p->b + k * p->ldb_bytes, N, row);
            for (int64_t n = 0; n < N; ++n) w[n * K + k] = row[n];
        }
        free(row);
    }
    if (p->w_round_f16) {
        for (int64_t i = 0; i < N * K; ++i) w[i] = orc_f16_to_f32(orc_f32_to_f16(w[i]));
    }
    for (int64_t m = m0; m < m1; ++m) {
        for (int64_t k = 0; k < K; ++k) {
            a[k] = p->a_f16 ? orc_f16_to_f32(((const uint16_t*)p->a)[m * p->lda + k])
                            : ((const float*)p->a)[m * p->lda + k];
        }
        for (int64_t n = 0; n < N; ++n) {
            const float* wr = w + n * K;
            float out;
            if (p->acc_f64) {
                double s = 0.0;
                for (int64_t k = 0; k < K; ++k) s += (double)a[k] * (double)wr[k];
                out = (float)s;
            } else {
                float s = 0.0f;
                for (int64_t k = 0; k < K; ++k) {
                    const float pr = a[k] * wr[k];
                    s += pr;
                }
                out = s;
            }
            if (p->c_f16) ((uint16_t*)p->c)[m * p->ldc + n] = orc_f32_to_f16(out);
            else ((float*)p->c)[m * p->ldc + n] = out;
        }
    }
    free(a);
    free(w);
}

/* ---------------------------------------------------------------------------
 * The fp output pass of the fp x q4_1 routes.
 *  - not gated: Linear / MatMul's fp epilogue order: bias, the pre-activation
 *    residual, clamp and activation (apply_epilogue, simd_epilogue.hpp:56-90),
 *    then the post-activation residual added to the destination-typed result
 *    (src/backend/cpu/matmul/linear.cpp:276-301: a compact temporary, then
 *    residual_add at :181-196);
 *  - gated: linear_gated_impl (linear.cpp:116-170): the GEMM with bias into a
 *    [rows, 2n] tile of the destination's type, then gated_combine_act
 *    (linear.cpp:84-114): act(gate) * (value + beta) with both halves clamped
 *    to +-limit when finite, Linear's epilogue, add_to accumulating onto the
 *    destination (tiled_map_simd's s_store_add, simd_kernel/tiled_map.hpp:
 *    40-66); the gate activation is gate_act_scalar (common/gate_combine.hpp:
 *    70-85).
 * ------------------------------------------------------------------------- */
static float gate_act_scalar(int32_t act, float g, float alpha)
{
    switch (act) {
    case ORC_ACT_SILU: return g / (1.0f + expf(-alpha * g));
    case ORC_ACT_GELU: return 0.5f * g * (1.0f + tanhf(0.7978845608028654f * (g + 0.044715f * g * g * g)));
    case ORC_ACT_RELU: return g > 0.0f ? g : 0.0f;
    case ORC_ACT_SIGMOID: return 1.0f / (1.0f + expf(-g));
    case ORC_ACT_TANH: return tanhf(g);
    default: return g;
    }
}

static float fp_round(int32_t f16, float x)
{
    return f16 ? orc_f16_to_f32(orc_f32_to_f16(x)) : x;
}

static float fp_load(int32_t f16, const void* base, int64_t i)
{
    return f16 ? orc_f16_to_f32(((const uint16_t*)base)[i]) : ((const float*)base)[i];
}

void orc_fp_out_pass(const orc_fp_out_t* p)
{
    for (int64_t r = 0; r < p->rows; ++r) {
        for (int64_t c = 0; c < p->n; ++c) {
            const int64_t oi = r * p->ld_out + c;
            const float beta = p->residual_pre ? 1.0f : p->beta;
            const int read_old = p->matmul_order ? beta != 0.0f : p->add_to;
            const float old = read_old ? fp_load(p->out_f16, p->out, oi) : 0.0f;
            const float bg = p->bias ? fp_load(p->out_f16, p->bias, c) : 0.0f;
            float y;
            if (p->matmul_order) {
                /* matmul_qblock_fused.cpp:106-142: C primed with beta old +
                 * bias in its own type (tile_scale_add_bias, separately
                 * rounded mul and add; matmul_helper.cpp:924-943) or scaled
                 * by beta (tile_scale), then alpha times the product joins it
                 * (mma_qblock.hpp:255-266), clamped, and the activation. */
                float init = 0.0f;
                if (p->bias) init = beta == 0.0f ? bg : fp_round(p->out_f16, old * beta + bg);
                else if (beta == 1.0f) init = old;
                else if (beta != 0.0f) init = fp_round(p->out_f16, old * beta);
                const float prod = p->alpha == 1.0f ? p->src[r * p->ld_src + c] : p->src[r * p->ld_src + c] * p->alpha;
                y = apply_act_fp(p->act, prod + init, p->min_clip, p->max_clip, p->act_alpha, p->act_beta);
            } else if (p->gated) {
                const float bv = p->bias ? fp_load(p->out_f16, p->bias, p->n + c) : 0.0f;
                float g = fp_round(p->out_f16, p->src[r * p->ld_src + c] + bg);
                float v = fp_round(p->out_f16, p->src[r * p->ld_src + p->n + c] + bv);
                if (isfinite(p->gate_limit)) {
                    g = fmaxf(fminf(g, p->gate_limit), -p->gate_limit);
                    v = fmaxf(fminf(v, p->gate_limit), -p->gate_limit);
                }
                y = apply_act_fp(p->act, gate_act_scalar(p->gate_act, g, p->gate_alpha) * (v + p->gate_beta),
                                 p->min_clip, p->max_clip, p->act_alpha, p->act_beta);
                /* the combined value is of the destination's type before it accumulates */
                if (p->add_to) y = old + fp_round(p->out_f16, y);
            } else {
                y = p->src[r * p->ld_src + c] + bg;
                if (p->add_to && p->residual_pre) y = y + old;
                y = apply_act_fp(p->act, y, p->min_clip, p->max_clip, p->act_alpha, p->act_beta);
                if (p->add_to && !p->residual_pre) y = fp_round(p->out_f16, y) + old;
            }
            if (p->out_f16) ((uint16_t*)p->out)[oi] = orc_f32_to_f16(y);
            else ((float*)p->out)[oi] = y;
        }
    }
}

/* ---------------------------------------------------------------------------
 * Seeded inputs: the xorshift128+ generator seeded through splitmix64 that the
 * reference's tests use (tests/common/random_tensor.hpp:18-57), so a seed names
 * the same data here as there.
 * ------------------------------------------------------------------------- */
static uint64_t splitmix64(uint64_t x)
{
    uint64_t z = x + 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

void orc_xs128_u64(uint64_t seed, int64_t count, uint64_t* out)
{
    uint64_t s0 = splitmix64(seed);
    uint64_t s1 = splitmix64(s0);
    for (int64_t i = 0; i < count; ++i) {
        uint64_t a = s0;
        const uint64_t b = s1;
        s0 = b;
        a ^= a << 23;
        s1 = a ^ b ^ (a >> 18) ^ (b >> 5);
        out[i] = s1 + b;
    }
}

/* ---------------------------------------------------------------------------
 * QuantizeLinear / DequantizeLinear over a flat row-major array of `count`
 * elements. Element i takes parameter j = (i / inner) % dim (per tensor: dim
 * 1; per token: inner = cols, dim = rows; per channel: inner = product of the
 * dims after the axis, dim = the axis extent), as
 * src/backend/cpu/quant_linear.cpp:97-118 maps the granularities onto the
 * kernel's per-row M x N shape.
 * ------------------------------------------------------------------------- */
static int64_t qdq_index(int64_t i, int64_t inner, int64_t dim)
{
    return dim <= 1 ? 0 : (i / inner) % dim;
}

/* src/backend/cpu/x86_64/quant.hpp:52-85 (vector body) and :162-167 (tail,
 * contracted to one FMA under -mfma): v = fma(x, 1/s, zp), rounded to nearest
 * even; the conversion of NaN or |v| >= 2^31 yields INT32_MIN, which the
 * saturating pack / clamp turn into qmin. */
void orc_quantize_linear(const void* x, int32_t x_f16, void* y, int32_t y_u8, int64_t count,
                         const float* scale, const int32_t* zero_point, int64_t inner, int64_t dim)
{
    const int32_t qmin = y_u8 ? 0 : -128, qmax = y_u8 ? 255 : 127;
    for (int64_t i = 0; i < count; ++i) {
        const float xv = x_f16 ? orc_f16_to_f32(((const uint16_t*)x)[i]) : ((const float*)x)[i];
        const int64_t j = qdq_index(i, inner, dim);
        const float inv = 1.0f / scale[j];
        const float zf = zero_point ? (float)zero_point[j] : 0.0f;
        const float v = fmaf(xv, inv, zf);
        int32_t q = INT32_MIN;
        if (fabsf(v) < 2147483648.0f) q = (int32_t)nearbyintf(v);
        if (q < qmin) q = qmin;
        if (q > qmax) q = qmax;
        if (y_u8) ((uint8_t*)y)[i] = (uint8_t)q;
        else ((int8_t*)y)[i] = (int8_t)q;
    }
}

/* src/backend/cpu/x86_64/quant.hpp:282-330: per row (here: per segment of
 * `segment` elements) the whole 16-element blocks compute fma(q, s, -zp*s) and
 * the last segment % 16 elements (q - zp) * s; f16 narrows the f32 result with
 * round to nearest even (the F16C conversion). */
void orc_dequantize_linear(const void* x, int32_t x_u8, void* y, int32_t y_f16, int64_t count,
                           const float* scale, const int32_t* zero_point, int64_t inner, int64_t dim,
                           int64_t segment)
{
    const int64_t body = segment - segment % 16;
    for (int64_t i = 0; i < count; ++i) {
        const int32_t q = x_u8 ? (int32_t)((const uint8_t*)x)[i] : (int32_t)((const int8_t*)x)[i];
        const int64_t j = qdq_index(i, inner, dim);
        const float s = scale[j];
        const float zf = zero_point ? (float)zero_point[j] : 0.0f;
        float v;
        if (i % segment < body) {
            const float nzs = -zf * s;
            v = fmaf((float)q, s, nzs);
        } else {
            const float d = (float)q - zf;
            v = d * s;
        }
        if (y_f16) ((uint16_t*)y)[i] = orc_f32_to_f16(v);
        else ((float*)y)[i] = v;
    }
}
