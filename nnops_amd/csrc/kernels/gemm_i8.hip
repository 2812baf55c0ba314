// Integer GEMM on gfx950: s8|u8 x s8 -> int32 accumulate on the int8 matrix
// cores, with the nnops output pass (compensate, bias, Relu, requant, or the
// float epilogue) applied to the accumulators in registers.
//
// Kernels
//   gemm_i8_mfma   M > 16: block tile BMxBN, k-step 64, A and B staged through
//                  LDS (k-contiguous rows padded to 80 B, so the 16-byte
//                  fragment reads of 8 consecutive rows hit disjoint banks),
//                  double-buffered global->register->LDS, v_mfma_i32_32x32x32_i8.
//                  Bound: MFMA (4096^3: arithmetic intensity ~2730 op/B).
//   gemv_i8_lds    4 < M <= 16, B [N][K]: 16 rows of B per block staged through
//                  LDS in 1 KiB row pieces, v_mfma_i32_16x16x64_i8.
//   gemv_i8_mfma   M <= 16 otherwise: one 16-column slice of B per block, K split over
//                  the block's 4 waves, fragments loaded straight from HBM into
//                  v_mfma_i32_16x16x64_i8 operands (no LDS on the weight path),
//                  partial tiles summed through LDS. Bound: HBM (weight bytes).
//   transpose_i8   [R][C] -> [C][R'] byte transpose through LDS (k-contiguous
//                  staging of a [K,N] B or a [K,M] A).
//   rowsum_i8      sum_k of each k-contiguous row (zero-point compensation).
//
// The reduction order of the int32 accumulate is irrelevant (integer addition
// is associative), so both kernels are bit-exact whatever the k split.
#include "common.hpp"

#include <type_traits>
#include <utility>

#include <algorithm>

namespace nnops_amd {
namespace {

constexpr int kBK = 64;        // k bytes per pipeline stage
constexpr int kLdsRow = 80;    // LDS row pitch (64 + 16 pad) in bytes

struct GemmI8Kern {
    const int8_t* a;     // [M][lda] k-contiguous
    const int8_t* b;     // [N][ldb] k-contiguous
    void* c;
    int m, n, k;
    int64_t lda, ldb, ldc_bytes;
    uint32_t a_xor;      // 0x80808080 when A is u8 (read as a - 128)
    EpiParams ep;
};

// ---------------------------------------------------------------------------
// 16-byte fragment loads (ALIGNED: base, pitch and K are multiples of 16).
// ---------------------------------------------------------------------------
template <bool ALIGNED>
__device__ __forceinline__ v4i load16(const int8_t* row, int k0, int K)
{
    if constexpr (ALIGNED) {
        if (k0 < K) {
            return *reinterpret_cast<const v4i*>(row + k0);
        }
        return v4i{0, 0, 0, 0};
    } else {
        uint32_t w[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            uint32_t v = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int kk = k0 + d * 4 + b;
                const uint32_t byte = kk < K ? (uint32_t)(uint8_t)row[kk] : 0u;
                v |= byte << (8 * b);
            }
            w[d] = v;
        }
        return v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
}

// A u8 operand is fed to the signed MFMA as a - 128 (flip the top bit of every
// byte); the epilogue adds 128 * sum_k b back through a_off. Padding bytes past
// K must stay 0 after the flip, which `valid` takes care of.
__device__ __forceinline__ v4i flip_u8(v4i v, uint32_t x, bool valid)
{
    if (x == 0u || !valid) {
        return v;
    }
    return v4i{(int)((uint32_t)v.x ^ x), (int)((uint32_t)v.y ^ x), (int)((uint32_t)v.z ^ x),
               (int)((uint32_t)v.w ^ x)};
}

// Unaligned path: bytes past K must read as 0 after the flip too, so flip per byte.
template <bool ALIGNED>
__device__ __forceinline__ v4i load16_a(const int8_t* row, int k0, int K, uint32_t x)
{
    v4i v = load16<ALIGNED>(row, k0, K);
    if (x == 0u) {
        return v;
    }
    if constexpr (ALIGNED) {
        return flip_u8(v, x, k0 < K);
    } else {
        uint32_t w[4] = {(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            uint32_t mask = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                if (k0 + d * 4 + b < K) {
                    mask |= 0x80u << (8 * b);
                }
            }
            w[d] ^= mask;
        }
        return v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
}

// ---------------------------------------------------------------------------
// Block-index mapping: consecutive logical tiles on one XCD (the hardware
// deals workgroups round-robin over the 8 XCDs), then grouped along M so the
// tiles resident on one XCD share A row panels and B column panels in its L2.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int& tm, int& tn)
{
    int bid = blockIdx.x;
    const int nb = gridDim.x;
    if ((nb & 7) == 0) {
        bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    }
    constexpr int G = 4;
    const int per_group = G * tiles_n;
    const int group = bid / per_group;
    const int first_m = group * G;
    const int gsize = min(tiles_m - first_m, G);
    const int in_group = bid - group * per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

// Stage loader: CA/CB 16-byte chunks per thread per 64-byte k stage. FULLK:
// K is a multiple of 64 and every row is 16-byte aligned, so no load needs a
// bound; otherwise chunks past K read as zero (ALIGNED or per byte).
template <int C, bool FULLK, bool ALIGNED, bool FLIP>
__device__ __forceinline__ void load_chunks(v4i (&r)[C], const int8_t* const (&src)[C],
                                            const int (&kc)[C], int k0, int K, uint32_t x)
{
#pragma unroll
    for (int i = 0; i < C; ++i) {
        if constexpr (FULLK) {
            r[i] = *reinterpret_cast<const v4i*>(src[i] + k0 + kc[i]);
            if constexpr (FLIP) {
                r[i] = flip_u8(r[i], x, true);
            }
        } else if constexpr (FLIP) {
            r[i] = load16_a<ALIGNED>(src[i], k0 + kc[i], K, x);
        } else {
            r[i] = load16<ALIGNED>(src[i], k0 + kc[i], K);
        }
    }
}

// ---------------------------------------------------------------------------
// Output pass shared by the MFMA kernels. One 32-row slab of the wave tile at a
// time goes through LDS (32x32 accumulator layout: lane holds column lane & 31,
// rows 8*(r/4) + 4*(lane/32) + (r%4)); then every lane owns 4 consecutive
// columns and walks the slab's rows, so the destination is written with packed
// 4-byte (s8/u8) or 16-byte (s32) stores, 4 rows in flight per lane.
//   EPI_S8   integer requant with row-uniform scales (no zero points, no
//            per-row tables): req = (s_a / s_out) * s_b[n] hoisted per column;
//   EPI_S32  raw accumulate + bias (+ Relu), no zero points;
//   EPI_GENERIC  everything else (compensation, per-row tables, float epilogue).
// The fast modes evaluate exactly the float operations epi_value does.
// ---------------------------------------------------------------------------
enum { EPI_GENERIC = 0, EPI_S8 = 1, EPI_S32 = 2 };

template <int FM, int FN, int TN, int EPI>
__device__ __forceinline__ void output_pass(const GemmI8Kern& p, v16i (&acc)[FM][FN], int32_t* slab,
                                            int row0, int col0, int lane)
{
    constexpr int kEpiPitch = TN + 4;
    constexpr int kColGroups = TN / 4;                   // 4-column groups per slab row
    constexpr int kRowStep = 64 / kColGroups;            // rows covered per pass of the wave
    constexpr int kRowsPerLane = 32 / kRowStep;
    static_assert(kColGroups * kRowStep == 64 && kRowsPerLane * kRowStep == 32, "slab walk");
    const EpiParams& ep = p.ep;
    const int cg = lane % kColGroups;
    const int rsub = lane / kColGroups;
    const int nb = col0 + cg * 4;                        // first of this lane's 4 columns
    EpiCol cols[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        cols[e] = epi_col(ep, min(nb + e, p.n - 1));
    }
    float req[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (EPI == EPI_S8) {
        const float row_k = __fdiv_rn(ep.s_a_scalar, ep.s_out);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            req[e] = __fmul_rn(row_k, cols[e].s_b);
        }
    }
    const bool relu = ep.act == NNOPS_ACT_RELU;
    const bool u8 = ep.out_kind == NNOPS_OUT_U8;
    const bool s32 = ep.out_kind == NNOPS_OUT_S32;
    const bool packed = !epi_is_fp(ep) && (nb + 3 < p.n) && (((uintptr_t)p.c & 15) == 0) &&
                        (s32 ? (p.ldc_bytes % 16 == 0) : (p.ldc_bytes % 4 == 0));
    // Fast modes (host-checked: N % 4 == 0, 16-byte-aligned C, pitch multiple
    // of the packed store, half-away rounding): branch-free per element.
    const int32_t relu_floor = relu ? 0 : INT32_MIN;
    const float zpf = (float)ep.zp_out;
    const float lo = __fsub_rn(u8 ? 0.0f : -128.0f, zpf);
    const float hi = __fsub_rn(u8 ? 255.0f : 127.0f, zpf);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                slab[row * kEpiPitch + j * 32 + (lane & 31)] = acc[i][j][r];
            }
        }
        __syncthreads();
        const int mbase = row0 + i * 32 + rsub;
        char* cbase = static_cast<char*>(p.c) + (int64_t)mbase * p.ldc_bytes +
                      (int64_t)nb * (s32 ? 4 : 1);
        const int64_t cstep = (int64_t)kRowStep * p.ldc_bytes;
#pragma unroll 4
        for (int t = 0; t < kRowsPerLane; ++t) {
            const int rr = rsub + t * kRowStep;
            const int m = mbase + t * kRowStep;
            char* cptr = cbase + t * cstep;
            if (m >= p.m || nb >= p.n) {
                continue;
            }
            const v4i raw = *reinterpret_cast<const v4i*>(&slab[rr * kEpiPitch + cg * 4]);
            if constexpr (EPI == EPI_S8) {
                uint32_t w = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int32_t v = max(raw[e] + cols[e].bias, relu_floor);
                    float x = __fmul_rn((float)v, req[e]);
                    x = __builtin_fminf(__builtin_fmaxf(x, lo), hi);
                    const int32_t q = (int32_t)round_half_away(x) + ep.zp_out;
                    w |= ((uint32_t)q & 0xffu) << (8 * e);
                }
                *reinterpret_cast<uint32_t*>(cptr) = w;
            } else if constexpr (EPI == EPI_S32) {
                v4i q;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    q[e] = max(raw[e] + cols[e].bias, relu_floor);
                }
                *reinterpret_cast<v4i*>(cptr) = q;
            } else {
                char* crow = static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes;
                const EpiRow row = epi_row(ep, m);
                if (packed && s32) {
                    int32_t q[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        q[e] = epi_value(ep, row, cols[e], raw[e], 0);
                    }
                    *reinterpret_cast<v4i*>(crow + (int64_t)nb * 4) = v4i{q[0], q[1], q[2], q[3]};
                } else if (packed) {
                    uint32_t old = 0;
                    if (ep.add_to) {
                        old = *reinterpret_cast<const uint32_t*>(crow + nb);
                    }
                    uint32_t w = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t ob = (old >> (8 * e)) & 0xffu;
                        const int32_t o = u8 ? (int32_t)ob : (int32_t)(int8_t)ob;
                        w |= ((uint32_t)epi_value(ep, row, cols[e], raw[e], o) & 0xffu) << (8 * e);
                    }
                    *reinterpret_cast<uint32_t*>(crow + nb) = w;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (nb + e < p.n) {
                            epi_store(ep, row, cols[e], raw[e], crow, nb + e);
                        }
                    }
                }
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Register output pass (EPI_S8 / EPI_S32): the element math runs in the MFMA
// accumulator layout (lane = one column, 4 consecutive rows per register
// group), then each 4x4 block is transposed across the lane quad with DPP so a
// lane holds 4 consecutive columns of one row and writes them with one packed
// store. No LDS round trip and no block barrier.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int quad_bcast(int v, int k)
{
    // quad_perm(k, k, k, k): every lane of the quad reads lane k
    switch (k) {
    case 0: return __builtin_amdgcn_mov_dpp(v, 0x00, 0xf, 0xf, true);
    case 1: return __builtin_amdgcn_mov_dpp(v, 0x55, 0xf, 0xf, true);
    case 2: return __builtin_amdgcn_mov_dpp(v, 0xaa, 0xf, 0xf, true);
    default: return __builtin_amdgcn_mov_dpp(v, 0xff, 0xf, 0xf, true);
    }
}

// Lane qi holds bytes (row 0..3) of column qi; returns (column 0..3) of row qi.
// Two exchange stages: with lane xor 1 (swapping lane bit 0 with byte bit 0),
// then with lane xor 2 (bit 1 with bit 1); each is one DPP move and one
// v_perm whose per-lane byte selectors (sel1, sel2) come from quad_sel.
// min(max(x, lo), hi) for lo <= hi in one v_med3_i32 (the compiler only forms
// it when it can prove lo <= hi).
__device__ __forceinline__ int32_t med3_i32(int32_t x, int32_t lo, int32_t hi)
{
    int32_t r;
    asm("v_med3_i32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(lo), "v"(hi));
    return r;
}

struct QuadSel {
    uint32_t s1, s2;
};

__device__ __forceinline__ QuadSel quad_sel(int qi)
{
    // v_perm_b32(hi = partner, lo = own, sel): selector byte b picks own.byte[b]
    // (b < 4) or partner.byte[b - 4]
    return QuadSel{(qi & 1) ? 0x03070105u : 0x06020400u, (qi & 2) ? 0x03020706u : 0x05040100u};
}

__device__ __forceinline__ uint32_t quad_transpose_bytes(uint32_t w, const QuadSel& qs)
{
    const uint32_t p1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)w, 0xb1, 0xf, 0xf, true);   // quad_perm(1,0,3,2)
    w = __builtin_amdgcn_perm(p1, w, qs.s1);
    const uint32_t p2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)w, 0x4e, 0xf, 0xf, true);   // quad_perm(2,3,0,1)
    return __builtin_amdgcn_perm(p2, w, qs.s2);
}

// 4x4 dword transpose across the quad: v[r] = (row r, column qi) in,
// v[c] = (row qi, column c) out. Two exchange stages (lane xor 1, xor 2).
__device__ __forceinline__ void quad_transpose_dwords(int32_t (&v)[4], int qi)
{
    const bool odd = qi & 1;
#pragma unroll
    for (int a = 0; a < 4; a += 2) {
        const int send = odd ? v[a] : v[a + 1];
        const int recv = __builtin_amdgcn_mov_dpp(send, 0xb1, 0xf, 0xf, true);  // quad_perm(1,0,3,2)
        if (odd) {
            v[a] = recv;
        } else {
            v[a + 1] = recv;
        }
    }
    const bool hi = qi & 2;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        const int send = hi ? v[a] : v[a + 2];
        const int recv = __builtin_amdgcn_mov_dpp(send, 0x4e, 0xf, 0xf, true);  // quad_perm(2,3,0,1)
        if (hi) {
            v[a] = recv;
        } else {
            v[a + 2] = recv;
        }
    }
}

// BIAS_IN_ACC: the accumulators started from bias[n], so it is not added again.
template <int FM, int FN, int EPI, bool BIAS_IN_ACC = false>
__device__ __forceinline__ void output_pass_regs(const GemmI8Kern& p, v16i (&acc)[FM][FN], int row0,
                                                 int col0, int lane)
{
    static_assert(EPI == EPI_S8 || EPI == EPI_S32, "register pass: fast modes only");
    const EpiParams& ep = p.ep;
    const int qi = lane & 3;
    const QuadSel qs = quad_sel(qi);
    const int colq = (lane & 31) & ~3;
    int32_t relu_floor = ep.act == NNOPS_ACT_RELU ? 0 : INT32_MIN;
    asm("" : "+s"(relu_floor));   // one max per element, not max + select on the flag
    const bool u8 = ep.out_kind == NNOPS_OUT_U8;
    const int32_t lo_i = (u8 ? 0 : -128) - ep.zp_out;
    const int32_t hi_i = (u8 ? 255 : 127) - ep.zp_out;
    const float row_k = __fdiv_rn(ep.s_a_scalar, ep.s_out);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int n_own = col0 + j * 32 + (lane & 31);       // column held before the transpose
        const EpiCol col = epi_col(ep, min(n_own, p.n - 1));
        const float req = __fmul_rn(row_k, col.s_b);
        const int n_st = col0 + j * 32 + colq;               // first column stored by this lane
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int m = row0 + i * 32 + 8 * g + 4 * (lane >> 5) + qi;
                char* cptr = static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes;
                if constexpr (EPI == EPI_S8) {
                    uint32_t q[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int32_t v = max(acc[i][j][4 * g + e] + (BIAS_IN_ACC ? 0 : col.bias), relu_floor);
                        const float x = __fmul_rn((float)v, req);
                        // round half away from zero (the conversion truncates, as
                        // trunc() would), then clamp in the integer domain: lo and
                        // hi are integers and rounding is monotonic, so this equals
                        // clamping x first; |x| past 2^31 saturates the conversion.
                        const int32_t r = (int32_t)__fadd_rn(x, __builtin_copysignf(0.5f, x));
                        q[e] = (uint32_t)(med3_i32(r, lo_i, hi_i) + ep.zp_out);
                    }
                    // low bytes of q[0..3] -> one word (0x0c selects a zero byte)
                    const uint32_t w01 = __builtin_amdgcn_perm(q[1], q[0], 0x0c0c0400u);
                    const uint32_t w23 = __builtin_amdgcn_perm(q[3], q[2], 0x04000c0cu);
                    const uint32_t w = quad_transpose_bytes(w01 | w23, qs);
                    if (m < p.m && n_st < p.n) {
                        *reinterpret_cast<uint32_t*>(cptr + n_st) = w;
                    }
                } else {
                    int32_t v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[e] = max(acc[i][j][4 * g + e] + (BIAS_IN_ACC ? 0 : col.bias), relu_floor);
                    }
                    quad_transpose_dwords(v, qi);
                    if (m < p.m && n_st < p.n) {
                        *reinterpret_cast<v4i*>(cptr + (int64_t)n_st * 4) = v4i{v[0], v[1], v[2], v[3]};
                    }
                }
            }
        }
    }
}

template <int BM, int BN, int WM, int WN, int WPE, bool FULLK, bool ALIGNED, bool FLIP, int EPI>
__global__ __launch_bounds__(WM * WN * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void gemm_i8_mfma(GemmI8Kern p)
{
    constexpr int T = WM * WN * 64;
    constexpr int TM = BM / WM;           // wave tile rows
    constexpr int TN = BN / WN;           // wave tile cols
    constexpr int FM = TM / 32;           // 32x32 fragments per wave
    constexpr int FN = TN / 32;
    constexpr int CA = BM * (kBK / 16) / T;   // 16-byte chunks per thread per stage
    constexpr int CB = BN * (kBK / 16) / T;
    static_assert(CA >= 1 && CB >= 1 && CA * T == BM * 4 && CB * T == BN * 4, "tile/threads");

    constexpr int kStageBytes = 2 * (BM + BN) * kLdsRow;
    constexpr int kEpiPitch = TN + 4;                      // int32 per staged output row
    constexpr int kEpiBytes = WM * WN * 32 * kEpiPitch * 4;
    static_assert(kEpiBytes <= kStageBytes, "epilogue staging must fit the stage buffers");
    __shared__ __attribute__((aligned(16))) int8_t lds_raw[kStageBytes];
    int8_t (*lds_a)[BM * kLdsRow] = reinterpret_cast<int8_t (*)[BM * kLdsRow]>(lds_raw);
    int8_t (*lds_b)[BN * kLdsRow] = reinterpret_cast<int8_t (*)[BN * kLdsRow]>(lds_raw + 2 * BM * kLdsRow);

    int tm, tn;
    tile_coords((p.m + BM - 1) / BM, (p.n + BN - 1) / BN, tm, tn);
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm0 = (wave / WN) * TM;
    const int wn0 = (wave % WN) * TN;

    // Per-thread stage chunks (rows past M/N are clamped: computed, never stored).
    const int8_t* a_src[CA];
    const int8_t* b_src[CB];
    int a_lds[CA], b_lds[CB], a_kc[CA], b_kc[CB];
#pragma unroll
    for (int i = 0; i < CA; ++i) {
        const int idx = tid + i * T;
        const int r = idx >> 2, c = idx & 3;
        a_src[i] = p.a + (int64_t)min(m0 + r, p.m - 1) * p.lda;
        a_kc[i] = c * 16;
        a_lds[i] = r * kLdsRow + c * 16;
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
        const int idx = tid + i * T;
        const int r = idx >> 2, c = idx & 3;
        b_src[i] = p.b + (int64_t)min(n0 + r, p.n - 1) * p.ldb;
        b_kc[i] = c * 16;
        b_lds[i] = r * kLdsRow + c * 16;
    }

    v4i ra[CA], rb[CB];
    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            acc[i][j] = v16i{0};
        }
    }

    const int frag_row = lane & 31;
    const int frag_k = (lane >> 5) * 16;
    const int kt = (p.k + kBK - 1) / kBK;

    load_chunks<CA, FULLK, ALIGNED, FLIP>(ra, a_src, a_kc, 0, p.k, p.a_xor);
    load_chunks<CB, FULLK, ALIGNED, false>(rb, b_src, b_kc, 0, p.k, 0u);
#pragma unroll
    for (int i = 0; i < CA; ++i) {
        *reinterpret_cast<v4i*>(&lds_a[0][a_lds[i]]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
        *reinterpret_cast<v4i*>(&lds_b[0][b_lds[i]]) = rb[i];
    }
    __syncthreads();

    for (int t = 0; t < kt; ++t) {
        const int cur = t & 1;
        const bool more = t + 1 < kt;
        if (more) {
            load_chunks<CA, FULLK, ALIGNED, FLIP>(ra, a_src, a_kc, (t + 1) * kBK, p.k, p.a_xor);
            load_chunks<CB, FULLK, ALIGNED, false>(rb, b_src, b_kc, (t + 1) * kBK, p.k, 0u);
        }
        const int8_t* la = &lds_a[cur][(wm0 + frag_row) * kLdsRow + frag_k];
        const int8_t* lb = &lds_b[cur][(wn0 + frag_row) * kLdsRow + frag_k];
#pragma unroll
        for (int ks = 0; ks < kBK; ks += 32) {
            v4i fa[FM], fb[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                fa[i] = *reinterpret_cast<const v4i*>(la + i * 32 * kLdsRow + ks);
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                fb[j] = *reinterpret_cast<const v4i*>(lb + j * 32 * kLdsRow + ks);
            }
#pragma unroll
            for (int i = 0; i < FM; ++i) {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (more) {
#pragma unroll
            for (int i = 0; i < CA; ++i) {
                *reinterpret_cast<v4i*>(&lds_a[cur ^ 1][a_lds[i]]) = ra[i];
            }
#pragma unroll
            for (int i = 0; i < CB; ++i) {
                *reinterpret_cast<v4i*>(&lds_b[cur ^ 1][b_lds[i]]) = rb[i];
            }
        }
        __syncthreads();
    }

    if constexpr (EPI == EPI_GENERIC) {
        output_pass<FM, FN, TN, EPI>(p, acc, reinterpret_cast<int32_t*>(lds_raw) + wave * 32 * kEpiPitch,
                                     m0 + wm0, n0 + wn0, lane);
    } else {
        output_pass_regs<FM, FN, EPI>(p, acc, m0 + wm0, n0 + wn0, lane);
    }
}

// ---------------------------------------------------------------------------
// Large-tile kernel with an asynchronous LDS ring (K % 64 == 0, 16-byte-aligned
// operands). Stages are filled by buffer_load_dwordx4 ... lds: each wave
// instruction writes 1 KiB of LDS contiguously (lane l -> bytes 16l..16l+15),
// i.e. 16 tile rows of 64 bytes, so the 16-byte chunk a lane fetches from HBM
// is chosen to land in a swizzled slot: row r's logical chunk c lives in slot
// c ^ ((r >> 2) & 3). A fragment read serves 16 lanes (16 consecutive rows,
// one logical chunk) per LDS cycle; with 64 four-byte banks those 16 reads land
// on 16 distinct 16-byte bank groups, so the read is conflict-free with no
// padding. NS stages are in flight, so each load has NS-1 k-steps of MFMA work
// to land before it is needed. The buffer form (32-bit offsets against a
// per-tile descriptor) costs fewer issue cycles than the 64-bit-address form.
//
// The MFMA takes the B fragment as its first operand, so the 32x32 accumulator
// holds C transposed: lane l owns output row (l & 31) and, in register group g,
// the 4 consecutive columns 8g + 4(l >> 5) + 0..3. Each lane therefore packs
// 4 output bytes (or one 16-byte int32 group) with no cross-lane transpose.
//
// Output modes:
//   RING_S8    fused requant (row-uniform s_a/s_out, per-column s_b, bias in
//              the accumulator init, Relu folded into the integer clamp);
//              bytes are staged per wave in LDS and written as 16-byte rows.
//   RING_S32   fused bias + Relu, int32 written straight from the accumulators.
//   RING_PART  raw int32 accumulators of this K split to a workspace slab;
//              gemm_i8_reduce sums the splits and runs the full output pass.
// ---------------------------------------------------------------------------
#define NNOPS_LPTR(x) ((__attribute__((address_space(3))) void*)(x))

// Buffer resource over [base, base + 2 GiB) with raw 32-bit offsets. The
// buffer builtins exist only in the device pass; the host pass sees a
// placeholder (kernels are never compiled for the host).
#if __HIP_DEVICE_COMPILE__
typedef __amdgpu_buffer_rsrc_t BufRsrc;
#else
struct BufRsrc {
    int w[4];
};
#endif

__device__ __forceinline__ BufRsrc buffer_rsrc(const void* base, int bytes = 0x7fffffff)
{
#if __HIP_DEVICE_COMPILE__
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
#else
    (void)base, (void)bytes;
    return BufRsrc{};
#endif
}

// ds_read_b64_tr_b8: each 16-lane group reads 16 rows of 8 bytes (one address
// per lane) and lane L of the group receives byte L & 7 of rows 2j + (L >> 3),
// j = 0..7. With lane i addressing row k0 + (i >> 1), columns c0 + 8 (i & 1)
// of a row-major byte tile, lane L receives column c0 + L at rows k0 .. k0 + 7:
// a k-contiguous fragment of a tile stored n-contiguous.
typedef int v2i __attribute__((ext_vector_type(2)));
__device__ __forceinline__ v2i lds_read_tr8(const int8_t* p)
{
#if __HIP_DEVICE_COMPILE__
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i*)(p));
#else
    (void)p;
    return v2i{0, 0};
#endif
}

// The same read as inline assembly, for loops whose LDS stages arrive by DMA:
// the compiler cannot tell the intrinsic's reads from the stages still in
// flight and puts a full vmcnt(0) before them, which drains the DMA ring every
// stage. The assembly is not tracked, so its results are pending until
// lds_tr8_ready ties them to an explicit lgkmcnt(0).
__device__ __forceinline__ v2i lds_read_tr8_asm(const int8_t* p)
{
    v2i r;
#if __HIP_DEVICE_COMPILE__
    const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) int8_t*)(p);
    asm volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(r) : "v"(a) : "memory");
#else
    (void)p;
    r = v2i{0, 0};
#endif
    return r;
}

// lgkmcnt(0) with the fragments built from lds_read_tr8_asm as in/out
// operands: their uses cannot move above it.
template <int N>
__device__ __forceinline__ void lds_tr8_ready_frags(v4i (&f)[N])
{
    static_assert(N == 1 || N == 2, "one or two fragments");
#if __HIP_DEVICE_COMPILE__
    if constexpr (N == 1) {
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]) : : "memory");
    } else {
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]) : : "memory");
    }
#else
    (void)f;
#endif
}

// Waits until at most S stages of L vector-memory operations each are in
// flight (S wave-uniform, clamped to MAXS).
template <int L, int MAXS>
__device__ __forceinline__ void wait_stages(int s)
{
    if constexpr (MAXS <= 0) {
        wait_vmcnt<0>();
    } else {
        if (s >= MAXS) {
            wait_vmcnt<MAXS * L>();
        } else {
            wait_stages<L, MAXS - 1>(s);
        }
    }
}

// Waits for every outstanding LDS read of the wave and makes the 16 values
// read by lds_read_tr8_asm depend on that wait, so no use moves above it.
__device__ __forceinline__ void lds_tr8_ready(v2i (&lo)[8], v2i (&hi)[8])
{
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(lo[0]), "+v"(lo[1]), "+v"(lo[2]), "+v"(lo[3]), "+v"(lo[4]), "+v"(lo[5]), "+v"(lo[6]),
                   "+v"(lo[7]), "+v"(hi[0]), "+v"(hi[1]), "+v"(hi[2]), "+v"(hi[3]), "+v"(hi[4]), "+v"(hi[5]),
                   "+v"(hi[6]), "+v"(hi[7])
                 :
                 : "memory");
#else
    (void)lo;
    (void)hi;
#endif
}

// Exchanges x's lanes 32..63 with y's lanes 0..31 (v_permlane32_swap): with
// x = a word of lane half h = 0 / 1 and y the same for another word, lane
// l < 32 ends with (x, y) = (x_l, x_{l+32}) and lane l + 32 with
// (y_l, y_{l+32}).
__device__ __forceinline__ void swap_half_waves(uint32_t& x, uint32_t& y)
{
#if __HIP_DEVICE_COMPILE__
    const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
    x = r[0];
    y = r[1];
#else
    (void)x, (void)y;
#endif
}

// 16 bytes per lane from base + voff + soff into LDS at lds + 16 * lane.
// AUX: the cache policy bits (2: non-temporal, for data read once).
template <int AUX = 0>
__device__ __forceinline__ void buffer_load_lds16(BufRsrc r, int8_t* lds, int voff, int soff)
{
#if __HIP_DEVICE_COMPILE__
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, NNOPS_LPTR(lds), 16, voff, soff, 0, AUX);
#else
    (void)r, (void)lds, (void)voff, (void)soff;
#endif
}

// Stores and loads with the sc1 cache policy: coherent at device scope (the
// lowering of an agent-scope atomic store / load) without a cache-wide fence;
// how the K splits of a one-launch kernel hand their partial sums over.
__device__ __forceinline__ void buffer_store4_sc1(BufRsrc r, int32_t v, int voff)
{
#if __HIP_DEVICE_COMPILE__
    __builtin_amdgcn_raw_buffer_store_b32(v, r, voff, 0, 16);
#else
    (void)r, (void)v, (void)voff;
#endif
}

__device__ __forceinline__ void buffer_store8_sc1(BufRsrc r, uint64_t v, int voff)
{
#if __HIP_DEVICE_COMPILE__
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2i, v), r, voff, 0, 16);
#else
    (void)r, (void)v, (void)voff;
#endif
}

__device__ __forceinline__ uint64_t buffer_load8_sc1(BufRsrc r, int voff)
{
#if __HIP_DEVICE_COMPILE__
    return __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 16));
#else
    (void)r, (void)voff;
    return 0;
#endif
}

__device__ __forceinline__ v4i buffer_load16_sc1(BufRsrc r, int voff)
{
#if __HIP_DEVICE_COMPILE__
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 16);
#else
    (void)r, (void)voff;
    return v4i{0, 0, 0, 0};
#endif
}

enum { RING_S8 = 0, RING_S32 = 1, RING_PART = 2, RING_FP = 3 };

// 16 zero bytes in global memory (never written): the address a lane loads
// from when its table value is absent, so the load needs no branch.
static __device__ __attribute__((aligned(16))) int32_t kZero16[4];

struct RingSplit {
    int splits;        // K ranges per output tile
    int kt_per;        // staged k steps per split (the last split takes the rest)
    int32_t* part;     // RING_PART: [splits][M][N] raw accumulators
    float row_k;       // gemm_i8_reduce_q: RN(s_a / s_out) and RN(1 / s_out), the
    float inv_out;     // host's correctly rounded f32 quotients (the device's bits)
    uint64_t* flag;    // gemv_i8_kn_tr: [column groups][splits] split-completion flags
    uint64_t epoch;    // the launch's flag value (graph replays repeat it), never 0
};

__device__ __forceinline__ void block_barrier()
{
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");  // no LDS access moves across the barrier
}

// Logical order: the hardware deals workgroups round-robin over the 8 XCDs,
// so consecutive logical ids are gathered on one XCD. Splits are outermost (a
// band of one XCD shares one K range of A), then tiles grouped 4 along M
// (neighbours share B column panels in that XCD's L2).
__device__ __forceinline__ void ring_coords(int tiles_m, int tiles_n, int& tm, int& tn, int& sp)
{
    int bid = blockIdx.x;
    const int nb = gridDim.x;
    if ((nb & 7) == 0) {
        bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    }
    const int tiles = tiles_m * tiles_n;
    sp = bid / tiles;
    bid -= sp * tiles;
    constexpr int G = 4;
    const int per_group = G * tiles_n;
    const int group = bid / per_group;
    const int first_m = group * G;
    const int gsize = min(tiles_m - first_m, G);
    const int in_group = bid - group * per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

// F16: the operands are f16 (the same byte staging: K, lda and ldb in bytes,
// a 16-byte lane fragment is 8 halves of v_mfma_f32_32x32x16_f16 as it is 16
// int8 of v_mfma_i32_32x32x32_i8), the accumulators f32; RING_FP then writes
// acc * s_a_scalar (alpha) and RING_PART the f32 partials' bits.
//
// TRB: B is [K,N] row-major (ldb its row pitch in bytes), staged as it lies: a
// stage holds BK k rows of BN bytes, 16-byte chunk c of row r in slot
// c ^ swzb(r), and the B fragments are built by lds_read_tr8 (two per
// fragment: k rows +0..7 and +8..15 of the lane's 16). No transposed copy.
template <int BM, int BN, int WM, int WN, int BK, int NS, int MODE, bool FLIP, bool F16 = false, bool TRB = false>
__global__ __launch_bounds__(WM * WN * 64)
__attribute__((amdgpu_waves_per_eu((WM * WN + 3) / 4, (WM * WN + 3) / 4)))
void gemm_i8_ring(GemmI8Kern p, RingSplit sk)
{
    static_assert(!F16 || MODE == RING_FP || MODE == RING_PART, "f16 operands: fp or partial outputs");
    static_assert(!TRB || !F16, "row-major B: int8 operands");
    constexpr int W = WM * WN;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int CPR = BK / 16;                  // 16-byte chunks per staged row
    constexpr int RPI = 1024 / BK;                // rows per 1 KiB load instruction
    constexpr int QA = BM / RPI / W;              // load instructions per wave per stage (A)
    constexpr int QB = BN / RPI / W;
    constexpr int L = QA + QB;                    // vector-memory ops per wave per stage
    // TRB rings of 128 rows and more: the transposed reads as untracked
    // assembly, per-stage counted waits to the end and step 0 peeled, so no
    // full vmcnt(0) drains the ring (4096^3: 73 -> 69 us; 333 x 4096 x
    // 14336: 46 -> 40 us). The 64 x 64 tiles (a handful of stages, latency
    // bound) and the [N,K] rings measured faster without.
    constexpr bool kTrAsm = TRB && BM >= 128;
    constexpr int S = BK / 32;                    // 32-k MFMA slices per stage
    constexpr int kStage = (BM + BN) * BK;
    constexpr int kPitch8 = TN + 16;              // staged byte row pitch: 2-way bank conflicts at most
    static_assert(BK == 64 || BK == 128, "stage depth");
    static_assert(QA * W * RPI == BM && QB * W * RPI == BN, "rows per stage");
    // TRB staging: 1024 / BN k rows per load instruction, CPRB chunks per row
    constexpr int RPIB = TRB ? 1024 / BN : 1;
    constexpr int CPRB = BN / 16;
    static_assert(!TRB || (1024 % BN == 0 && BN >= 64 && (BK / RPIB) == QB * W), "row-major B staging");
    static_assert(FM * 32 == TM && FN * 32 == TN, "wave tile");
    static_assert(W * TM * kPitch8 <= NS * kStage, "byte staging fits the ring");
    static_assert(NS >= 2 && (NS - 1) * L < 64, "vmcnt range");
    static_assert(MODE == RING_PART || !FLIP, "u8 A needs the compensating output pass");

    __shared__ __attribute__((aligned(1024))) int8_t ring[NS * kStage];
    // the output pass's per-column scales, staged at the start (their load
    // latency then hides behind the first stage's) where the LDS holds them
    constexpr bool kSbl = (MODE == RING_S8 || MODE == RING_FP) && NS * kStage + BN * 4 <= 160 * 1024;
    __shared__ __attribute__((aligned(16))) float sbl[kSbl ? BN : 4];
    // RING_FP: the bias in the destination's type, widened to f32, likewise
    constexpr bool kBl = MODE == RING_FP && kSbl && NS * kStage + BN * 8 <= 160 * 1024;
    __shared__ __attribute__((aligned(16))) float biasl[kBl ? BN : 4];

    int tm, tn, sp;
    ring_coords(ceil_div(p.m, BM), ceil_div(p.n, BN), tm, tn, sp);
    const int m0 = tm * BM, n0 = tn * BN;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm0 = (wave / WN) * TM, wn0 = (wave % WN) * TN;
    const int kt0 = sp * sk.kt_per;
    const int kt = (sp == sk.splits - 1) ? p.k / BK - kt0 : sk.kt_per;

    // Staged rows are BK bytes; chunk c of row r sits in slot c ^ swz(r), so
    // the 16 rows a fragment read serves per LDS cycle hit 16 distinct 16-byte
    // bank groups (BK = 64: 4 rows per 256 bytes, swz = (r >> 2) & 3;
    // BK = 128: 2 rows per 256 bytes, swz = (r >> 1) & 7).
    auto swz = [](int r) { return BK == 64 ? ((r >> 2) & 3) : ((r >> 1) & 7); };
    // TRB: a transposed read serves 8 k rows x two 16-byte chunks per 32
    // lanes; rows sharing a 256-byte bank row (256 / BN of them) keep their
    // slots, and the bank rows' 8 slot pairs differ in slot bits 1.., so the
    // 16 chunks fall in 16 distinct 16-byte bank groups.
    auto swzb = [](int r) { return ((r / (BN >= 256 ? 1 : 256 / BN)) & (CPRB / 2 - 1)) << 1; };

    // Descriptors over this tile's row panels from this split's first k; rows
    // past M/N are clamped to the last row (computed, never stored).
    const BufRsrc rsa = buffer_rsrc(p.a + (int64_t)m0 * p.lda + (int64_t)kt0 * BK);
    // TRB: the descriptor ends at B's last byte, so chunks past column N of
    // the last k row read 0 (earlier rows' read the next row: never stored)
    const BufRsrc rsb = TRB ? buffer_rsrc(p.b + (int64_t)kt0 * BK * p.ldb + n0,
                                          (int)((int64_t)(p.k - kt0 * BK - 1) * p.ldb + (p.n - n0)))
                            : buffer_rsrc(p.b + (int64_t)n0 * p.ldb + (int64_t)kt0 * BK);
    int a_off[QA], b_off[QB];
#pragma unroll
    for (int q = 0; q < QA; ++q) {
        const int r = (wave * QA + q) * RPI + lane / CPR;
        const int c = (lane % CPR) ^ swz(r);
        a_off[q] = min(r, p.m - 1 - m0) * (int)p.lda + c * 16;
    }
#pragma unroll
    for (int q = 0; q < QB; ++q) {
        if constexpr (TRB) {
            const int r = (wave * QB + q) * RPIB + lane / CPRB;
            const int c = (lane % CPRB) ^ swzb(r);
            b_off[q] = r * (int)p.ldb + c * 16;
        } else {
            const int r = (wave * QB + q) * RPI + lane / CPR;
            const int c = (lane % CPR) ^ swz(r);
            b_off[q] = min(r, p.n - 1 - n0) * (int)p.ldb + c * 16;
        }
    }
    const int b_step = TRB ? BK * (int)p.ldb : BK;     // bytes from one stage's B rows to the next's
    auto issue = [&](int s) {
        int8_t* base = ring + (s % NS) * kStage;
#pragma unroll
        for (int q = 0; q < QA; ++q) {
            buffer_load_lds16(rsa, base + (wave * QA + q) * 1024, a_off[q], s * BK);
        }
#pragma unroll
        for (int q = 0; q < QB; ++q) {
            buffer_load_lds16(rsb, base + BM * BK + (wave * QB + q) * 1024, b_off[q], s * b_step);
        }
    };

    // Accumulators (transposed layout), initialised after the first stage loads.
    std::conditional_t<F16, v16f, v16i> acc[FM][FN];

    // Fragment reads of slice ks: row (lane & 31) of each 32-row fragment,
    // logical chunk 2 ks + (lane >> 5).
    const int fr = lane & 31;
    auto frag = [&](const int8_t* st, int row, int ks) {
        const int c = (2 * ks + (lane >> 5)) ^ swz(row);
        return *reinterpret_cast<const v4i*>(st + row * BK + c * 16);
    };
    // TRB: the B fragment of columns col .. col + 31 at slice ks from the
    // row-major stage: lane (group g, index i) addresses k row 32 ks + 16 (g
    // >> 1) + (i >> 1) (+8 for the second read), columns col + 16 (g & 1) +
    // 8 (i & 1); lane l receives column col + (l & 31) at k 32 ks + 16 (l >>
    // 5) + 0..15, the layout of the A fragments.
    const int tr_k = 16 * (lane >> 5) + ((lane & 15) >> 1);
    const int tr_c = 16 * ((lane >> 4) & 1) + 8 * (lane & 1);
    auto frag_tr = [&](const int8_t* stb, int col, int ks) {
        const int k0 = 32 * ks + tr_k;
        const int c = col + tr_c;
        const int8_t* plo = stb + k0 * BN + (((c >> 4) ^ swzb(k0)) << 4) + (c & 15);
        const int8_t* phi = stb + (k0 + 8) * BN + (((c >> 4) ^ swzb(k0 + 8)) << 4) + (c & 15);
        if constexpr (kTrAsm) {
            // untracked reads: step() ties them to an lgkmcnt(0) before their use
            const v2i lo = lds_read_tr8_asm(plo);
            const v2i hi = lds_read_tr8_asm(phi);
            return v4i{lo.x, lo.y, hi.x, hi.y};
        } else {
            const v2i lo = lds_read_tr8(plo);
            const v2i hi = lds_read_tr8(phi);
            return v4i{lo.x, lo.y, hi.x, hi.y};
        }
    };
    auto read_frags = [&](const int8_t* st, int ks, v4i (&fa)[FM], v4i (&fb)[FN]) {
        if constexpr (TRB) {
            fb[0] = frag_tr(st + BM * BK, wn0, ks);
        } else {
            fb[0] = frag(st + BM * BK, wn0 + fr, ks);
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            fa[i] = frag(st, wm0 + i * 32 + fr, ks);
        }
#pragma unroll
        for (int j = 1; j < FN; ++j) {
            if constexpr (TRB) {
                fb[j] = frag_tr(st + BM * BK, wn0 + j * 32, ks);
            } else {
                fb[j] = frag(st + BM * BK, wn0 + j * 32 + fr, ks);
            }
        }
    };
    auto mfma_all = [&](v4i (&fa)[FM], const v4i (&fb)[FN]) {
        if constexpr (FLIP) {  // u8 A enters the signed MFMA as a - 128
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                fa[i] ^= v4i{(int)0x80808080u, (int)0x80808080u, (int)0x80808080u, (int)0x80808080u};
            }
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                if constexpr (F16) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, fb[j]),
                                                                      __builtin_bit_cast(v8h, fa[i]), acc[i][j], 0,
                                                                      0, 0);
                } else {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[j], fa[i], acc[i][j], 0, 0, 0);
                }
            }
        }
    };
    // One fragment read after each of the first FM + FN MFMAs, so every read
    // has part of a slice of matrix work to land before it is needed; with
    // loads, they go on the last MFMAs of the slice.
    constexpr int NR = FM + (TRB ? 2 : 1) * FN;     // LDS reads per slice
    auto schedule = [&](bool loads) {
#pragma unroll
        for (int q = 0; q < FM * FN; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (q < NR) {
                if (q + 1 < FM * FN) {
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                } else {
                    // the last MFMA takes the reads left over
                    __builtin_amdgcn_sched_group_barrier(0x100, NR - FM * FN + 1, 0);
                }
            }
            if (loads && q >= FM * FN - L && q - (FM * FN - L) < L) {
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
        }
    };

    // The output pass's column tables: bias[n] (whose values start the
    // accumulators of the fused modes), the staged s_b and fp bias.
    // kTrAsm: bias[n] and s_b are loaded before the first stages are issued
    // and used after (with step 0 peeled the first use then waits for these
    // loads alone); every lane loads unconditionally, from a 16-byte zero
    // stand-in where a value is absent, since a load under a branch is waited
    // for where the branch joins. Elsewhere they follow the first stages
    // (measured as fast or faster there).
    const int32_t* const zero16 = kZero16;
    v4i bpre[kTrAsm ? FN : 1][4];
    const int nsb = n0 + 4 * (int)threadIdx.x;
    const bool sb_live = kTrAsm && kSbl && threadIdx.x < BN / 4 && p.ep.s_b != nullptr && nsb < p.n;
    v4f sbpre = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (kTrAsm) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                bpre[j][g] = v4i{0, 0, 0, 0};
                if constexpr (MODE != RING_PART) {
                    const int n = n0 + wn0 + j * 32 + 8 * g + 4 * (lane >> 5);
                    const bool live = p.ep.bias != nullptr && n < p.n;
                    bpre[j][g] = *reinterpret_cast<const v4i*>(live ? p.ep.bias + n : zero16);
                }
            }
        }
        if constexpr (kSbl) {
            sbpre = *reinterpret_cast<const v4f*>(sb_live ? p.ep.s_b + nsb : reinterpret_cast<const float*>(zero16));
        }
        // keep those loads ahead of the stages
        asm volatile("" ::: "memory");
    }

    // Ring: stage s goes to slot s % NS; nothing is issued past this split's
    // last stage, so the vmcnt waits count only the stages really in flight.
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) {
        if (s < kt) {
            issue(s);
        }
    }
    // Accumulators (transposed layout); the fused modes start from bias[n].
#pragma unroll
    for (int j = 0; j < FN && F16; ++j) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            acc[i][j] = std::conditional_t<F16, v16f, v16i>{0};
        }
    }
#pragma unroll
    for (int j = 0; j < FN && !F16; ++j) {
        int32_t b0[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            v4i bv = v4i{0, 0, 0, 0};
            if constexpr (kTrAsm) {
                bv = bpre[j][g];
            } else if constexpr (MODE != RING_PART) {
                const int n = n0 + wn0 + j * 32 + 8 * g + 4 * (lane >> 5);
                if (p.ep.bias != nullptr && n < p.n) {
                    bv = *reinterpret_cast<const v4i*>(p.ep.bias + n);
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                b0[4 * g + e] = bv[e];
            }
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc[i][j][r] = b0[r];
            }
        }
    }
    if constexpr (kSbl) {
        if (threadIdx.x < BN / 4) {
            const int n = n0 + 4 * (int)threadIdx.x;
            v4f v = v4f{p.ep.s_b_scalar, p.ep.s_b_scalar, p.ep.s_b_scalar, p.ep.s_b_scalar};
            if constexpr (kTrAsm) {
                if (sb_live) {
                    v = sbpre;
                }
            } else if (p.ep.s_b != nullptr && n < p.n) {
                v = *reinterpret_cast<const v4f*>(p.ep.s_b + n);
            }
            *reinterpret_cast<v4f*>(&sbl[4 * threadIdx.x]) = v;
        }
    }
    if constexpr (kBl) {
        if (threadIdx.x >= BN / 4 && threadIdx.x < BN / 2) {
            const int t = (int)threadIdx.x - BN / 4;
            const int n = n0 + 4 * t;
            v4f v = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            if (p.ep.bias_fp != nullptr && n < p.n) {
                if (p.ep.out_kind == NNOPS_OUT_F16) {
                    const _Float16* b16 = static_cast<const _Float16*>(p.ep.bias_fp) + n;
                    v = v4f{(float)b16[0], (float)b16[1], (float)b16[2], (float)b16[3]};
                } else {
                    v = *reinterpret_cast<const v4f*>(static_cast<const float*>(p.ep.bias_fp) + n);
                }
            }
            *reinterpret_cast<v4f*>(&biasl[4 * t]) = v;
        }
    }
    // stage 0 landed; the others issued (up to NS - 2) may stay in flight
    if constexpr (kTrAsm) {
        wait_stages<L, NS - 2>(min(kt, NS - 1) - 1);
    } else if (kt >= NS - 1) {
        wait_vmcnt<(NS - 2) * L>();
    } else {
        wait_vmcnt<0>();
    }
    block_barrier();

    v4i f0a[FM], f0b[FN], f1a[FM], f1b[FN];
    read_frags(ring, 0, f0a, f0b);
    // One stage: stage t+NS-1 is issued into the slot read in step t-1 (freed
    // by that step's barrier); slice ks runs on the matrix cores while slice
    // ks+1's fragments load; after the last slice, wait for stage t+1 (its
    // later stages may stay in flight) and for every wave's reads of stage t
    // (lgkmcnt, then the barrier), then read slice 0 of stage t+1.
    auto step = [&](int t) {
        const int8_t* st = ring + (t % NS) * kStage;
        const bool more = t + NS - 1 < kt;
        if (more) {
            issue(t + NS - 1);
        }
#pragma unroll
        for (int ks = 0; ks < S; ++ks) {
            v4i (&ca)[FM] = (ks & 1) ? f1a : f0a;
            v4i (&cb)[FN] = (ks & 1) ? f1b : f0b;
            v4i (&na)[FM] = (ks & 1) ? f0a : f1a;
            v4i (&nb)[FN] = (ks & 1) ? f0b : f1b;
            if constexpr (kTrAsm) {
                lds_tr8_ready_frags(cb);
            }
            if (ks + 1 < S) {
                read_frags(st, ks + 1, na, nb);
                mfma_all(ca, cb);
                schedule(false);
            } else {
                mfma_all(ca, cb);
                if constexpr (kTrAsm) {
                    // stage t + 1 landed; the ones after it may stay in
                    // flight (all issued: kt - 2 - t of them)
                    wait_stages<L, NS - 2>(more ? NS - 2 : kt - 2 - t);
                } else if (more) {
                    wait_vmcnt<(NS - 2) * L>();
                } else {
                    wait_vmcnt<0>();
                }
                __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's reads of stage t are done
                block_barrier();
                if (t + 1 < kt) {
                    read_frags(ring + ((t + 1) % NS) * kStage, 0, na, nb);
                }
            }
        }
    };
    // kTrAsm: step 0 outside the loop (the accumulators start from loaded
    // values, and a loop that uses loaded values while issuing loads of its
    // own gets a full vmcnt(0) before it)
    int t0 = 0;
    if constexpr (kTrAsm) {
        if (kt > 0) {
            step(0);
        }
        t0 = 1;
    }
    for (int t = t0; t < kt; ++t) {
        step(t);
    }
    // The output pass's per-column scales: from the LDS copy staged at the
    // start, or else a lane's 8 loads issued together with one wait. They are
    // not read during the last stage: that would raise the loop's register
    // peak past the 256 of two waves per SIMD.
    const EpiParams& ep = p.ep;
    v4f sbp[FN][4];
    if constexpr (MODE == RING_S8 || MODE == RING_FP) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int nl = wn0 + j * 32 + 8 * g + 4 * (lane >> 5);
                if constexpr (kSbl) {
                    sbp[j][g] = *reinterpret_cast<const v4f*>(&sbl[nl]);
                } else {
                    sbp[j][g] = v4f{ep.s_b_scalar, ep.s_b_scalar, ep.s_b_scalar, ep.s_b_scalar};
                    if (ep.s_b != nullptr && n0 + nl < p.n) {
                        sbp[j][g] = *reinterpret_cast<const v4f*>(ep.s_b + n0 + nl);
                    }
                }
            }
        }
    }
    __syncthreads();   // every wave is done with the ring before it is reused for staging

    if constexpr (MODE == RING_S8) {
        // Requant in the transposed layout: per lane 4 consecutive columns of
        // one row per register group. Relu is folded into the clamp: with
        // req >= 0 a negative v gives r <= 0 and Relu's 0 gives r = 0, so
        // raising the low bound to 0 yields the same code; with req < 0 the high
        // bound drops to 0 instead. The integer clamp equals nnops' float clamp
        // before rounding (the bounds are integers and rounding is monotonic).
        const bool relu = ep.act == NNOPS_ACT_RELU;
        const bool u8 = ep.out_kind == NNOPS_OUT_U8;
        const int32_t lo_i = (u8 ? 0 : -128) - ep.zp_out;
        const int32_t hi_i = (u8 ? 255 : 127) - ep.zp_out;
        const float row_k = __fdiv_rn(ep.s_a_scalar, ep.s_out);
        // the whole [BM][BN] byte tile staged at once where the ring holds it,
        // so the stores are whole rows of the tile (BN bytes: whole 128-byte
        // lines) rather than each wave's TN-byte segments
        constexpr int kWholeP = BN + 16;
        constexpr bool kWhole = BM * kWholeP <= NS * kStage && (BN % 128) == 0 && (BM * BN / 16) % (W * 64) == 0;
        constexpr int kSP = kWhole ? kWholeP : kPitch8;
        int8_t* stage8 = kWhole ? ring + wm0 * kSP + wn0 : ring + wave * (TM * kPitch8);
        // Two instructions per element are dropped where the parameters
        // allow: with Relu, only the rounding of values on the unclamped side
        // of 0 reaches the output (the other side clamps to 0 whichever way it
        // rounds), so the half-away addend is the column's constant
        // +-0.5 (the sign of req) instead of copysign(0.5, x); and a zero
        // output zero point needs no add.
        // Each lane packs one row's 4 columns per register group g (columns
        // 8g + 4h .. +3, h = lane / 32); a permlane32 swap of groups (0, 2)
        // and (1, 3) then gives lane h the row's 16 contiguous columns 16h ..
        // 16h + 15 of the fragment, written to the stage as one 16-byte LDS
        // store (four 4-byte stores with 2-way bank conflicts before: the
        // largest part of the output pass).
        auto requant = [&](auto relu_c, auto zp_c) {
            constexpr bool kRelu = decltype(relu_c)::value;
            constexpr bool kZp = decltype(zp_c)::value;
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                uint32_t w[FM][4];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const v4f sb = sbp[j][g];
                    float req[4], half[4];
                    int32_t lo[4], hi[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        req[e] = __fmul_rn(row_k, sb[e]);
                        lo[e] = (kRelu && req[e] >= 0.0f) ? max(lo_i, 0) : lo_i;
                        hi[e] = (kRelu && !(req[e] >= 0.0f)) ? min(hi_i, 0) : hi_i;
                        half[e] = req[e] >= 0.0f ? 0.5f : -0.5f;
                    }
#pragma unroll
                    for (int i = 0; i < FM; ++i) {
                        uint32_t q[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float x = __fmul_rn((float)acc[i][j][4 * g + e], req[e]);
                            // round half away from zero: the conversion truncates as trunc() does
                            const float h = kRelu ? half[e] : __builtin_copysignf(0.5f, x);
                            const int32_t r = (int32_t)__fadd_rn(x, h);
                            q[e] = (uint32_t)(kZp ? med3_i32(r, lo[e], hi[e]) + ep.zp_out : med3_i32(r, lo[e], hi[e]));
                        }
                        w[i][g] = __builtin_amdgcn_perm(q[1], q[0], 0x0c0c0400u) |
                                  __builtin_amdgcn_perm(q[3], q[2], 0x04000c0cu);
                    }
                }
#pragma unroll
                for (int i = 0; i < FM; ++i) {
                    swap_half_waves(w[i][0], w[i][2]);
                    swap_half_waves(w[i][1], w[i][3]);
                    const v4i v = v4i{(int)w[i][0], (int)w[i][2], (int)w[i][1], (int)w[i][3]};
                    *reinterpret_cast<v4i*>(stage8 + (i * 32 + (lane & 31)) * kSP + j * 32 + 16 * (lane >> 5)) = v;
                }
            }
        };
        using TrueC = std::integral_constant<bool, true>;
        using FalseC = std::integral_constant<bool, false>;
        if (relu && ep.zp_out == 0) {
            requant(TrueC{}, FalseC{});
        } else if (relu) {
            requant(TrueC{}, TrueC{});
        } else if (ep.zp_out == 0) {
            requant(FalseC{}, FalseC{});
        } else {
            requant(FalseC{}, TrueC{});
        }
        if constexpr (kWhole) {
            __syncthreads();
            // 16-byte chunks of whole tile rows, wave w taking rows w, w + W, ...
            constexpr int CPRW = BN / 16;
#pragma unroll
            for (int q = 0; q < BM * CPRW / (W * 64); ++q) {
                const int idx = (q * W + wave) * 64 + lane, r = idx / CPRW, c = idx % CPRW;
                const int m = m0 + r, n = n0 + c * 16;
                const v4i v = *reinterpret_cast<const v4i*>(ring + r * kSP + c * 16);
                if (m < p.m && n < p.n) {
                    char* cptr = static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes + n;
                    __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(cptr));
                }
            }
            return;
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        // 16-byte row chunks of the wave tile (host-checked: N % 16 == 0,
        // 16-byte-aligned C and pitch)
        constexpr int CPR = TN / 16;
#pragma unroll
        for (int q = 0; q < TM * CPR / 64; ++q) {
            const int idx = q * 64 + lane, r = idx / CPR, c = idx % CPR;
            const int m = m0 + wm0 + r, n = n0 + wn0 + c * 16;
            const v4i v = *reinterpret_cast<const v4i*>(stage8 + r * kPitch8 + c * 16);
            if (m < p.m && n < p.n) {
                char* cptr = static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes + n;
                __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(cptr));
            }
        }
    } else if constexpr (MODE == RING_FP) {
        // f32 / f16 destination, plain operands (no zero points) and an
        // identity or Relu activation (host-checked): f = v * (s_a * s_b[n])
        // [+ bias[n]] [+ C_old before / after the clip], clip, Relu -- the
        // operation order of the generic pass (epi_value_fp). Host-checked:
        // N % 4 == 0, 16-byte-aligned C and pitch.
        const bool f16 = ep.out_kind == NNOPS_OUT_F16;
        const bool relu = ep.act == NNOPS_ACT_RELU;
        const bool pre = ep.add_to && ep.residual_pre, post = ep.add_to && !ep.residual_pre;
        // per 4-column group (j, g): the columns' scales and bias, loaded once
        // for the FM row fragments that share them
        struct ColFp {
            v4f sb, bias;
            int n;
        };
        auto col_fp = [&](int j, int g) {
            ColFp cp;
            cp.n = n0 + wn0 + j * 32 + 8 * g + 4 * (lane >> 5);
            cp.sb = sbp[j][g];
            cp.bias = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (kBl) {
                cp.bias = *reinterpret_cast<const v4f*>(&biasl[cp.n - n0]);
            } else if (cp.n < p.n && ep.bias_fp != nullptr) {
                if (f16) {
                    const _Float16* b16 = static_cast<const _Float16*>(ep.bias_fp) + cp.n;
                    cp.bias = v4f{(float)b16[0], (float)b16[1], (float)b16[2], (float)b16[3]};
                } else {
                    cp.bias = *reinterpret_cast<const v4f*>(static_cast<const float*>(ep.bias_fp) + cp.n);
                }
            }
            return cp;
        };
        // the 4 values of (i, j, g) for this lane: row wm0 + 32 i + (lane & 31),
        // columns cp.n .. + 3
        // CLIP: a finite clip range (the default -inf / +inf clip is the
        // identity for every value, NaN included, and is left out)
        // FORM (host-known) > 0: no residual and no clip, so the value is
        // v * (s_a * s_b[n]) [+ bias[n]] [Relu] with no per-element branches
        // (1: neither, 2: bias, 3: Relu, 4: both), the general order's
        // operations; 0: the general pass
        auto values = [&](int i, int j, int g, const ColFp& cp, float sa, auto clip_c, auto form_c) {
            constexpr bool kClip = decltype(clip_c)::value;
            constexpr int kForm = decltype(form_c)::value;
            constexpr bool kPlain = kForm > 0;
            const int n = cp.n;
            const int m = m0 + wm0 + i * 32 + (lane & 31);
            v4f o = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            if (n >= p.n || m >= p.m) {
                return o;
            }
            v4f old = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            if (!kPlain && ep.add_to) {
                const char* cptr = static_cast<const char*>(p.c) + (int64_t)m * p.ldc_bytes + (int64_t)n * (f16 ? 2 : 4);
                if (f16) {
                    const _Float16* o16 = reinterpret_cast<const _Float16*>(cptr);
                    old = v4f{(float)o16[0], (float)o16[1], (float)o16[2], (float)o16[3]};
                } else {
                    old = *reinterpret_cast<const v4f*>(cptr);
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float f = __fmul_rn((float)acc[i][j][4 * g + e], __fmul_rn(sa, cp.sb[e]));
                if constexpr (kPlain) {
                    if constexpr (kForm == 2 || kForm == 4) {
                        f = __fadd_rn(f, cp.bias[e]);
                    }
                    if constexpr (kForm == 3 || kForm == 4) {
                        f = f > 0.0f ? f : 0.0f;
                    }
                    o[e] = f;
                    continue;
                }
                if (ep.bias_fp != nullptr) {
                    f = __fadd_rn(f, cp.bias[e]);
                }
                if (pre) {
                    f = __fadd_rn(f, old[e]);
                }
                if constexpr (kClip) {
                    f = f < ep.min_clip ? ep.min_clip : f;
                    f = ep.max_clip < f ? ep.max_clip : f;
                }
                if (relu) {
                    f = f > 0.0f ? f : 0.0f;
                }
                if (post) {
                    if (f16) {
                        f = (float)(_Float16)f;
                    }
                    f = __fadd_rn(f, old[e]);
                }
                o[e] = f;
            }
            return o;
        };
        float sa_i[FM];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int m = min(m0 + wm0 + i * 32 + (lane & 31), p.m - 1);
            sa_i[i] = ep.s_a != nullptr ? ep.s_a[m] : ep.s_a_scalar;
        }
        if constexpr (W * TM * 128 <= NS * kStage) {
            // Staged through LDS so the global stores are 16-byte chunks
            // along rows (whole 128-byte lines per 8 lanes): per wave a
            // [TM][128-byte] tile of one slab of columns (32 f32 or 64 f16),
            // entries of 4 columns at slot q ^ (row % groups) in the row.
            int8_t* tile = ring + wave * (TM * 128);
            auto slab = [&](auto esz_c, auto clip_c, auto form_c) {
                constexpr int ESZ = decltype(esz_c)::value;          // output element bytes
                constexpr int SC = (TN < 128 / ESZ) ? TN : 128 / ESZ; // columns per slab
                constexpr int GPS = SC / 4;                          // 4-column entries per slab row
                constexpr int E = 4 * ESZ;                           // entry bytes
                constexpr int RB = GPS * E;                          // slab row bytes
                constexpr int CPRW = RB / 16;                        // 16-byte chunks per row
#pragma unroll
                for (int s0 = 0; s0 < TN / SC; ++s0) {
#pragma unroll
                    for (int jj = 0; jj < SC / 32; ++jj) {
                        const int j = s0 * (SC / 32) + jj;
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            const int q = jj * 8 + 2 * g + (lane >> 5);
                            const ColFp cp = col_fp(j, g);
#pragma unroll
                            for (int i = 0; i < FM; ++i) {
                                const int r = i * 32 + (lane & 31);
                                const v4f o = values(i, j, g, cp, sa_i[i], clip_c, form_c);
                                int8_t* dst = tile + r * RB + ((q ^ (r % GPS)) * E);
                                if constexpr (ESZ == 4) {
                                    *reinterpret_cast<v4f*>(dst) = o;
                                } else {
                                    _Float16 h[4] = {(_Float16)o[0], (_Float16)o[1], (_Float16)o[2], (_Float16)o[3]};
                                    uint2 w;
                                    __builtin_memcpy(&w, h, 8);
                                    *reinterpret_cast<uint2*>(dst) = w;
                                }
                            }
                        }
                    }
                    __builtin_amdgcn_wave_barrier();
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                    for (int t = 0; t < TM * CPRW / 64; ++t) {
                        const int idx = t * 64 + lane, r = idx / CPRW, cc = idx % CPRW;
                        const int m = m0 + wm0 + r;
                        const int n = n0 + wn0 + s0 * SC + cc * (16 / ESZ);
                        v4i v;
                        if constexpr (ESZ == 4) {
                            v = *reinterpret_cast<const v4i*>(tile + r * RB + ((cc ^ (r % GPS)) * E));
                        } else {
                            const uint2 lo = *reinterpret_cast<const uint2*>(tile + r * RB + (((2 * cc) ^ (r % GPS)) * E));
                            const uint2 hi = *reinterpret_cast<const uint2*>(tile + r * RB + (((2 * cc + 1) ^ (r % GPS)) * E));
                            v = v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
                        }
                        if (m < p.m && n < p.n) {
                            char* cptr = static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes + (int64_t)n * ESZ;
                            if (n + 16 / ESZ <= p.n) {
                                __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(cptr));
                            } else {
                                // a row's last group of 4 columns (N % 8 == 4, f16)
                                *reinterpret_cast<uint2*>(cptr) = uint2{(uint32_t)v.x, (uint32_t)v.y};
                            }
                        }
                    }
                    __builtin_amdgcn_wave_barrier();
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                }
            };
            using TrueC = std::integral_constant<bool, true>;
            using FalseC = std::integral_constant<bool, false>;
            const bool clip = !(ep.min_clip == -__builtin_inff() && ep.max_clip == __builtin_inff());
            using F0 = std::integral_constant<int, 0>;
            const bool fast = !clip && !ep.add_to;
            const int form = !fast ? 0 : 1 + (ep.bias_fp != nullptr ? 1 : 0) + (relu ? 2 : 0);
            auto run = [&](auto esz_c) {
                if (form == 1) {
                    slab(esz_c, FalseC{}, std::integral_constant<int, 1>{});
                } else if (form == 2) {
                    slab(esz_c, FalseC{}, std::integral_constant<int, 2>{});
                } else if (form == 3) {
                    slab(esz_c, FalseC{}, std::integral_constant<int, 3>{});
                } else if (form == 4) {
                    slab(esz_c, FalseC{}, std::integral_constant<int, 4>{});
                } else if (clip) {
                    slab(esz_c, TrueC{}, F0{});
                } else {
                    slab(esz_c, FalseC{}, F0{});
                }
            };
            if (f16) {
                run(std::integral_constant<int, 2>{});
            } else {
                run(std::integral_constant<int, 4>{});
            }
        } else {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int n = n0 + wn0 + j * 32 + 8 * g + 4 * (lane >> 5);
                    const ColFp cp = col_fp(j, g);
#pragma unroll
                    for (int i = 0; i < FM; ++i) {
                        const int m = m0 + wm0 + i * 32 + (lane & 31);
                        if (m >= p.m || n >= p.n) {
                            continue;
                        }
                        const v4f o = values(i, j, g, cp, sa_i[i], std::integral_constant<bool, true>{},
                                             std::integral_constant<int, 0>{});
                        char* cptr = static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes + (int64_t)n * (f16 ? 2 : 4);
                        if (f16) {
                            _Float16 h[4] = {(_Float16)o[0], (_Float16)o[1], (_Float16)o[2], (_Float16)o[3]};
                            uint2 w;
                            __builtin_memcpy(&w, h, 8);
                            *reinterpret_cast<uint2*>(cptr) = w;
                        } else {
                            *reinterpret_cast<v4f*>(cptr) = o;
                        }
                    }
                }
            }
        }
    } else {
        // int32 groups (host-checked: N % 4 == 0, 16-byte-aligned rows),
        // staged through the ring so every store is a 16-byte piece of a
        // whole tile row: 32 lanes write one row's BN * 4 bytes. Straight
        // from the accumulator layout a store instruction would touch 32 rows
        // with 32 bytes each, which writes at a fraction of the HBM rate
        // (config 5's 22 MB of partials: 9.6 us against 3 us for the same
        // bytes in row pieces). Passes of PI fragment rows per wave row keep
        // the staged slab within the ring.
        const int32_t floor_v = (MODE == RING_S32 && ep.act == NNOPS_ACT_RELU) ? 0 : INT32_MIN;
        char* cbase;
        int64_t ld;
        if constexpr (MODE == RING_S32) {
            cbase = static_cast<char*>(p.c);
            ld = p.ldc_bytes;
        } else {
            cbase = reinterpret_cast<char*>(sk.part + (int64_t)sp * p.m * p.n);
            ld = (int64_t)p.n * 4;
        }
        constexpr int kRowB = BN * 4 + 16;            // staged row pitch: rows 16 bytes apart in the banks
        constexpr int PI = (WM * FM * 32 * kRowB <= NS * kStage) ? FM
                           : (FM % 2 == 0 && WM * (FM / 2) * 32 * kRowB <= NS * kStage) ? FM / 2 : 1;
        static_assert(WM * PI * 32 * kRowB <= NS * kStage, "int32 staging fits the ring");
        constexpr int kCPR = BN / 4;                  // 16-byte chunks per tile row
        constexpr int kRows = WM * PI * 32;           // staged rows per pass
        static_assert((kRows * kCPR) % (W * 64) == 0, "whole chunks per thread");
        const int wmi = wave / WN;
#pragma unroll
        for (int pass = 0; pass < FM / PI; ++pass) {
#pragma unroll
            for (int ii = 0; ii < PI; ++ii) {
                const int i = pass * PI + ii;
                const int sr = (wmi * PI + ii) * 32 + (lane & 31);
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    v16i a;
                    if constexpr (F16) {
                        a = __builtin_bit_cast(v16i, acc[i][j]);
                    } else {
                        a = acc[i][j];
                    }
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        v4i v;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            v[e] = F16 ? a[4 * g + e] : max(a[4 * g + e], floor_v);
                        }
                        const int col = wn0 + j * 32 + 8 * g + 4 * (lane >> 5);
                        *reinterpret_cast<v4i*>(ring + sr * kRowB + col * 4) = v;
                    }
                }
            }
            __syncthreads();
#pragma unroll
            for (int q = 0; q < kRows * kCPR / (W * 64); ++q) {
                const int idx = (q * W + wave) * 64 + lane;
                const int sr = idx / kCPR, cc = idx % kCPR;
                const int m = m0 + (sr / (PI * 32)) * TM + (pass * PI + (sr / 32) % PI) * 32 + (sr & 31);
                const int n = n0 + cc * 4;
                const v4i v = *reinterpret_cast<const v4i*>(ring + sr * kRowB + cc * 16);
                if (m < p.m && n < p.n) {
                    // the int32 destination is written once; the partials are
                    // read back by the reduce, so they keep the default policy
                    if constexpr (MODE == RING_S32) {
                        __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(cbase + (int64_t)m * ld + (int64_t)n * 4));
                    } else {
                        *reinterpret_cast<v4i*>(cbase + (int64_t)m * ld + (int64_t)n * 4) = v;
                    }
                }
            }
            if (pass + 1 < FM / PI) {
                __syncthreads();
            }
        }
    }
}

// The output pass of 4 consecutive columns nb..nb+3 of row m: its row and
// column constants and the residual word, loaded before the raw sums arrive
// (out4_prepare), then the pass itself (out4_store).
struct Out4 {
    EpiRow row;
    EpiCol cols[4];
    uint32_t oldw;
    char* crow;
    int8_t* c8;
    bool word8;
};

__device__ __forceinline__ Out4 out4_prepare(const GemmI8Kern& p, int m, int nb)
{
    const EpiParams& ep = p.ep;
    Out4 o{};
    o.crow = static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes;
    o.c8 = reinterpret_cast<int8_t*>(o.crow) + nb;
    o.word8 = !epi_is_fp(ep) && ep.out_kind != NNOPS_OUT_S32 && ((uintptr_t)o.c8 & 3) == 0;
    o.row = epi_row(ep, m);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        o.cols[e] = epi_col(ep, nb + e);
    }
    if (o.word8 && ep.add_to) {
        o.oldw = *reinterpret_cast<const uint32_t*>(o.c8);
    }
    return o;
}

__device__ __forceinline__ void out4_store(const GemmI8Kern& p, const Out4& o, int nb, v4i raw)
{
    const EpiParams& ep = p.ep;
    const bool u8 = ep.out_kind == NNOPS_OUT_U8;
    if (epi_is_fp(ep)) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            epi_store(ep, o.row, o.cols[e], raw[e], o.crow, nb + e);
        }
        return;
    }
    if (ep.out_kind == NNOPS_OUT_S32) {
        int32_t* c32 = reinterpret_cast<int32_t*>(o.crow) + nb;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            c32[e] = epi_value(ep, o.row, o.cols[e], raw[e], 0);
        }
        return;
    }
    if (o.word8) {
        // one 4-byte read of the residual (in out4_prepare) and one 4-byte store
        uint32_t outw = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t ob = (o.oldw >> (8 * e)) & 0xffu;
            const int32_t old = u8 ? (int32_t)ob : (int32_t)(int8_t)ob;
            outw |= ((uint32_t)epi_value(ep, o.row, o.cols[e], raw[e], old) & 0xffu) << (8 * e);
        }
        *reinterpret_cast<uint32_t*>(o.c8) = outw;
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int32_t old = ep.add_to ? (u8 ? (int32_t)((const uint8_t*)o.c8)[e] : (int32_t)o.c8[e]) : 0;
        o.c8[e] = (int8_t)epi_value(ep, o.row, o.cols[e], raw[e], old);
    }
}

// Sum of the K-split partial accumulators and the full output pass
// (compensation, bias, Relu, requant or the float epilogue, add_to). TPG
// threads share a group of 4 consecutive columns of a row (N % 4 == 0), each
// summing every TPG-th split with its loads in flight together, then combine
// with lane shuffles; the first of them runs the output pass. TPG = 16 suits
// many splits of a small output (each thread's loads in one round trip), TPG =
// 1 a few splits of a large one.
template <int TPG>
__global__ __launch_bounds__(256) void gemm_i8_reduce(GemmI8Kern p, RingSplit sk)
{
    const int groups = p.n / 4;
    const int64_t gid = ((int64_t)blockIdx.x * 256 + threadIdx.x) / TPG;
    const int j = threadIdx.x % TPG;
    const bool in = gid < (int64_t)p.m * groups;
    const int m = in ? (int)(gid / groups) : 0;
    const int nb = in ? (int)(gid - (int64_t)m * groups) * 4 : 0;
    const int64_t slab = (int64_t)p.m * p.n;
    const int32_t* src = sk.part + (int64_t)m * p.n + nb;
    // the output pass's constants and the residual word, loaded with the
    // partials rather than after them
    Out4 o{};
    if (in && j == 0) {
        o = out4_prepare(p, m, nb);
    }
    v4i raw = v4i{0, 0, 0, 0};
    if (in) {
        int s = j;
        for (; s + 3 * TPG < sk.splits; s += 4 * TPG) {
            const v4i x0 = *reinterpret_cast<const v4i*>(src + s * slab);
            const v4i x1 = *reinterpret_cast<const v4i*>(src + (s + TPG) * slab);
            const v4i x2 = *reinterpret_cast<const v4i*>(src + (s + 2 * TPG) * slab);
            const v4i x3 = *reinterpret_cast<const v4i*>(src + (s + 3 * TPG) * slab);
            raw += (x0 + x1) + (x2 + x3);
        }
        for (; s < sk.splits; s += TPG) {
            raw += *reinterpret_cast<const v4i*>(src + s * slab);
        }
    }
    if constexpr (TPG > 1) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
#pragma unroll
            for (int o = 1; o < TPG; o <<= 1) {
                raw[e] += __shfl_xor(raw[e], o);
            }
        }
    }
    if (!in || j != 0) {
        return;
    }
    out4_store(p, o, nb, raw);
}

// The same sum and output pass for s8 / u8 destinations with row-uniform
// parameters (per-tensor s_a, s_out and zp_out, no zero-point terms, 16-byte
// aligned tables, 4-byte aligned destination rows), with the activation,
// float epilogue and residual order fixed at compile time: every load a
// thread needs (its splits' partial groups, the column tables and the
// residual word) is issued before the first is used, and the arithmetic is
// straight-line. One thread per 4-column group, grid.y walking the rows (no
// per-thread division for the row); element for element the operations of
// epi_value, so the bytes equal gemm_i8_reduce's.
template <int ACT, bool FEP, bool ADD, bool PRE>
__global__ __launch_bounds__(256) void gemm_i8_reduce_q(GemmI8Kern p, RingSplit sk)
{
    const EpiParams& ep = p.ep;
    const int nb = ((int)blockIdx.x * 256 + (int)threadIdx.x) * 4;
    if (nb >= p.n) {
        return;
    }
    const v4f sb = ep.s_b != nullptr ? *reinterpret_cast<const v4f*>(ep.s_b + nb)
                                     : v4f{ep.s_b_scalar, ep.s_b_scalar, ep.s_b_scalar, ep.s_b_scalar};
    const v4i bias = ep.bias != nullptr ? *reinterpret_cast<const v4i*>(ep.bias + nb) : v4i{0, 0, 0, 0};
    const bool u8 = ep.out_kind == NNOPS_OUT_U8;
    const bool even = ep.round_even != 0;
    const float row_k = sk.row_k;
    const float inv_out = sk.inv_out;
    const bool clip = !(ep.min_clip == -__builtin_inff() && ep.max_clip == __builtin_inff());
    const int64_t slab = (int64_t)p.m * p.n;
    for (int m = (int)blockIdx.y; m < p.m; m += (int)gridDim.y) {
        const int32_t* src = sk.part + (int64_t)m * p.n + nb;
        v4i raw = v4i{0, 0, 0, 0};
        int s = 0;
        for (; s + 3 < sk.splits; s += 4) {
            const v4i x0 = *reinterpret_cast<const v4i*>(src + s * slab);
            const v4i x1 = *reinterpret_cast<const v4i*>(src + (s + 1) * slab);
            const v4i x2 = *reinterpret_cast<const v4i*>(src + (s + 2) * slab);
            const v4i x3 = *reinterpret_cast<const v4i*>(src + (s + 3) * slab);
            raw += (x0 + x1) + (x2 + x3);
        }
        for (; s < sk.splits; ++s) {
            raw += *reinterpret_cast<const v4i*>(src + s * slab);
        }
        int8_t* c8 = static_cast<int8_t*>(p.c) + (int64_t)m * p.ldc_bytes + nb;
        uint32_t oldw = 0;
        if constexpr (ADD) {
            oldw = *reinterpret_cast<const uint32_t*>(c8);
        }
        uint32_t outw = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            int32_t v = raw[e] + bias[e];
            int32_t q;
            if constexpr (!FEP) {
                if constexpr (ACT == NNOPS_ACT_RELU) {
                    v = v < 0 ? 0 : v;
                }
                q = requant_clamped(__fmul_rn((float)v, __fmul_rn(row_k, sb[e])), ep.zp_out, u8, even);
            } else {
                float f = __fmul_rn((float)v, __fmul_rn(ep.s_a_scalar, sb[e]));
                float res = 0.0f;
                if constexpr (ADD) {
                    const uint32_t ob = (oldw >> (8 * e)) & 0xffu;
                    const int32_t old = u8 ? (int32_t)ob : (int32_t)(int8_t)ob;
                    res = __fmul_rn((float)(old - ep.zp_out), ep.s_out);
                    if constexpr (PRE) {
                        f = __fadd_rn(f, res);
                    }
                }
                if (clip) {   // the default -inf / +inf clip is the identity
                    f = f < ep.min_clip ? ep.min_clip : f;
                    f = ep.max_clip < f ? ep.max_clip : f;
                }
                if constexpr (ACT == NNOPS_ACT_RELU) {
                    f = f > 0.0f ? f : 0.0f;
                } else if constexpr (ACT == NNOPS_ACT_GELU) {
                    f = gelu_tanh(f);
                }
                if constexpr (ADD && !PRE) {
                    f = __fadd_rn(f, res);
                }
                q = requant_clamped(div_by_fixed(f, ep.s_out, inv_out), ep.zp_out, u8, even);
            }
            outw |= ((uint32_t)q & 0xffu) << (8 * e);
        }
        *reinterpret_cast<uint32_t*>(c8) = outw;
    }
}

// ---------------------------------------------------------------------------
// GEMV / skinny GEMM, M <= 16.
// ---------------------------------------------------------------------------
template <int U, bool ALIGNED>
__global__ __launch_bounds__(256) void gemv_i8_mfma(GemmI8Kern p)
{
    constexpr int W = 4;                  // waves per block, splitting K
    __shared__ v4i red[W - 1][64];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * 16;
    const int col = min(n0 + (lane & 15), p.n - 1);
    const int arow = lane & 15;
    const bool a_live = arow < p.m;
    const int kg = (lane >> 4) * 16;
    const int8_t* brow = p.b + (int64_t)col * p.ldb;
    const int8_t* a_row = p.a + (int64_t)(a_live ? arow : 0) * p.lda;

    const int ksteps = (p.k + 63) / 64;
    v4i acc = {0, 0, 0, 0};
    for (int s0 = wave * U; s0 < ksteps; s0 += W * U) {
        v4i fb[U], fa[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k0 = (s0 + u) * 64 + kg;
            const bool live = (s0 + u) < ksteps;
            fb[u] = live ? load16<ALIGNED>(brow, k0, p.k) : v4i{0, 0, 0, 0};
            fa[u] = (live && a_live) ? load16_a<ALIGNED>(a_row, k0, p.k, p.a_xor)
                                     : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[u], fb[u], acc, 0, 0, 0);
        }
    }

    if (wave > 0) {
        red[wave - 1][lane] = acc;
    }
    __syncthreads();
    if (wave != 0) {
        return;
    }
#pragma unroll
    for (int w = 0; w < W - 1; ++w) {
        acc += red[w][lane];
    }
    // 16x16 layout: lane holds column (lane & 15), rows 4*(lane/16) + r.
    const int n = n0 + (lane & 15);
    if (n >= p.n) {
        return;
    }
    const EpiCol c = epi_col(p.ep, n);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = 4 * (lane >> 4) + r;
        if (m < p.m) {
            const EpiRow row = epi_row(p.ep, m);
            char* crow = static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes;
            epi_store(p.ep, row, c, acc[r], crow, n);
        }
    }
}

// ---------------------------------------------------------------------------
// Skinny GEMM, 4 < M <= 16, B k-contiguous ([N][K], 16-byte aligned rows):
// one block per 16 rows of B (16 output columns), its W waves splitting K in
// 1 KiB pieces (wave w: k = 1024 w + 1024 W j). Each wave moves its 16 rows x
// 1 KiB of B into LDS with one direct-to-LDS load per row (1 KiB of whole
// cache lines per instruction, where the register-fed GEMV's fragment loads
// fetch 64-byte half lines) while its A fragments (16 rows x 1 KiB, from L2)
// go to registers; then 16 v_mfma_i32_16x16x64_i8 read B back from LDS (row
// pitch 1040 bytes: a fragment read's 16 rows fall in distinct bank groups).
// K tails: A reads zero past K; B reads past the block's last row come back
// zero from the buffer's range check. Bound: HBM (the B stream).
// ---------------------------------------------------------------------------
template <int W>
__global__ __launch_bounds__(W * 64) void gemv_i8_lds(GemmI8Kern p)
{
    constexpr int KW = 1024;                         // k bytes per wave piece
    constexpr int PITCH = KW + 16;                   // LDS row pitch
    constexpr int T = KW / 64;                       // MFMAs per piece
    __shared__ __attribute__((aligned(16))) int8_t stage[W][16 * PITCH];
    __shared__ v4i red[W - 1][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * 16;
    const int rows = min(16, p.n - n0);
    const int64_t span = (int64_t)(rows - 1) * p.ldb + p.k;
#if __HIP_DEVICE_COMPILE__
    const BufRsrc rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(p.b + (int64_t)n0 * p.ldb), 0,
                                                         (int)span, 0x00020000);
#else
    (void)span;
    const BufRsrc rs{};
#endif
    const int arow = lane & 15;
    const bool a_live = arow < p.m;
    const int8_t* a_row = p.a + (int64_t)(a_live ? arow : 0) * p.lda;
    const int kq = (lane >> 4) * 16;
    int8_t* st = stage[wave];
    // A plain int32 destination (no zero-point terms) takes only the bias and
    // Relu; its bias word is loaded now, off the output pass's critical path
    const bool plain32 = p.ep.out_kind == NNOPS_OUT_S32 && !p.ep.compensate;
    const int n_out = n0 + (lane & 15);
    int32_t bias_n = 0;
    if (plain32 && wave == 0 && p.ep.bias != nullptr && n_out < p.n) {
        bias_n = p.ep.bias[n_out];
    }
    // the general output pass's column and row constants, likewise up front
    EpiCol col{};
    EpiRow rws[4]{};
    if (!plain32 && wave == 0 && n_out < p.n) {
        col = epi_col(p.ep, n_out);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            rws[r] = epi_row(p.ep, min(4 * (lane >> 4) + r, p.m - 1));
        }
    }

    v4i acc = {0, 0, 0, 0};
    for (int kb = wave * KW; kb < p.k; kb += W * KW) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            buffer_load_lds16<2>(rs, st + r * PITCH, (int)((int64_t)r * p.ldb) + kb + lane * 16, 0);
        }
        v4i fa[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            fa[t] = a_live ? load16_a<true>(a_row, kb + 64 * t + kq, p.k, p.a_xor) : v4i{0, 0, 0, 0};
        }
        wait_vmcnt<0>();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const v4i fb = *reinterpret_cast<const v4i*>(st + arow * PITCH + 64 * t + kq);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[t], fb, acc, 0, 0, 0);
        }
        // the next piece's loads overwrite this stage: its reads must be done
        __builtin_amdgcn_s_waitcnt(0xc07f);
        asm volatile("" ::: "memory");
    }

    if (wave > 0) {
        red[wave - 1][lane] = acc;
    }
    __syncthreads();
    if (wave != 0) {
        return;
    }
#pragma unroll
    for (int w = 0; w < W - 1; ++w) {
        acc += red[w][lane];
    }
    // 16x16 layout: lane holds column (lane & 15), rows 4*(lane/16) + r.
    const int n = n_out;
    if (n >= p.n) {
        return;
    }
    if (plain32) {
        const bool relu = p.ep.act == NNOPS_ACT_RELU;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 4 * (lane >> 4) + r;
            if (m < p.m) {
                const int32_t v = acc[r] + bias_n;
                reinterpret_cast<int32_t*>(static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes)[n] =
                    (relu && v < 0) ? 0 : v;
            }
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = 4 * (lane >> 4) + r;
        if (m < p.m) {
            char* crow = static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes;
            epi_store(p.ep, rws[r], col, acc[r], crow, n);
        }
    }
}

// ---------------------------------------------------------------------------
// Row GEMV, M <= 4, B k-contiguous ([N][K]). A wave owns R consecutive rows of
// B; lane l reads the 16-byte chunks k = 16*(l + 64c), so every wave load
// instruction streams 1 KiB of one row contiguously (non-temporal: the
// weights are read once). Dots on v_dot4_i32_i8, A kept in registers per
// 4 KiB k block, cross-lane sum at the end. Bound: HBM.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int wave_sum(int v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        v += __shfl_xor(v, off, 64);
    }
    return v;
}

template <int MT, int R, bool FLIP, int WPB = 4, int SPLIT = 1>
__global__ __launch_bounds__(WPB * 64) void gemv_i8_rows(GemmI8Kern p)
{
    // SPLIT > 1: SPLIT consecutive waves share one row (R = 1), each taking an
    // interleaved 1/SPLIT of its 1 KiB k chunks; partial sums meet in LDS.
    static_assert(SPLIT == 1 || R == 1, "split rows are single rows");
    static_assert(WPB % SPLIT == 0, "a row's waves share a block");
    constexpr int C = 4;                       // 16-byte chunks per lane per row per k block
    __shared__ int part[SPLIT > 1 ? WPB : 1][R * MT];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sub = wave % SPLIT;
    const int n0 = ((blockIdx.x * WPB + wave) / SPLIT) * R;
    const bool row_live = n0 < p.n;
    const int8_t* brow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        brow[r] = p.b + (int64_t)min(n0 + r, p.n - 1) * p.ldb;
    }
    int acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            acc[r][m] = 0;
        }
    }
    for (int kb = 0; kb < p.k; kb += 64 * 16 * C) {
        v4i w[R][C], a[MT][C];
        // weights first (the HBM stream is the long pole), then A from cache
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const int k = kb + (lane + 64 * c) * 16;
            const bool live = row_live && (c % SPLIT == sub) && k < p.k;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                w[r][c] = live ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(brow[r] + k))
                               : v4i{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const int k = kb + (lane + 64 * c) * 16;
            const bool live = row_live && (c % SPLIT == sub) && k < p.k;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const int mm = min(m, p.m - 1);
                v4i x = live ? *reinterpret_cast<const v4i*>(p.a + (int64_t)mm * p.lda + k) : v4i{0, 0, 0, 0};
                if constexpr (FLIP) {
                    x = flip_u8(x, p.a_xor, live);
                }
                a[m][c] = x;
            }
        }
#pragma unroll
        for (int c = 0; c < C; ++c) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    int s = acc[r][m];
                    s = __builtin_amdgcn_sdot4(a[m][c].x, w[r][c].x, s, false);
                    s = __builtin_amdgcn_sdot4(a[m][c].y, w[r][c].y, s, false);
                    s = __builtin_amdgcn_sdot4(a[m][c].z, w[r][c].z, s, false);
                    s = __builtin_amdgcn_sdot4(a[m][c].w, w[r][c].w, s, false);
                    acc[r][m] = s;
                }
            }
        }
    }
    int mine = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int v = wave_sum(acc[r][m]);
            if (lane == r * MT + m) {
                mine = v;
            }
        }
    }
    if constexpr (SPLIT > 1) {
        if (lane < R * MT) {
            part[wave][lane] = mine;
        }
        __syncthreads();
        if (sub != 0) {
            return;
        }
        if (lane < R * MT) {
#pragma unroll
            for (int q = 1; q < SPLIT; ++q) {
                mine += part[wave + q][lane];
            }
        }
    }
    if (row_live && lane < R * MT) {
        const int r = lane / MT, m = lane % MT;
        const int n = n0 + r;
        if (n < p.n && m < p.m) {
            char* crow = static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes;
            epi_store(p.ep, epi_row(p.ep, m), epi_col(p.ep, n), mine, crow, n);
        }
    }
}

// ---------------------------------------------------------------------------
// Column GEMV, M <= 16, B n-contiguous ([K][N], the MatMul weight without
// transpose_b), consumed in place. Lane l of a wave owns CPL consecutive
// columns (the launch takes CPL = 4: one 4-byte load per row; the template
// also takes 16), so every wave load streams 64 * CPL contiguous bytes of one row. Four
// rows k..k+3 are transposed in registers (two v_perm per column) into one
// dword of 4 k-bytes per column, which v_dot4 multiplies with A[m][k..k+3]
// read through the scalar cache (A is uniform across the wave). Split s of S
// takes k-quads [s Q / S, (s + 1) Q / S) of a column chunk, and the W waves of
// its workgroup equal parts of that range, summed by LDS atomic adds (W = 4
// or 8); the workgroups write raw
// int32 partials that gemm_i8_reduce sums and passes through the output pass.
// (Meeting the splits inside the kernel, the last-arriving split summing the
// others through device-coherent loads, measured slower: the handoff costs
// more than the second launch.) Bound: HBM.
// ---------------------------------------------------------------------------
typedef const __attribute__((address_space(4))) int32_t* ScalarI32Ptr;

struct KnSplit {
    int chunks;       // column chunks of 64 * CPL
};

// 4 rows (one dword each, byte c = column c) -> 4 column dwords (byte i = row i)
__device__ __forceinline__ void transpose4x4_bytes(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3,
                                                   uint32_t (&col)[4])
{
    const uint32_t t0 = __builtin_amdgcn_perm(r1, r0, 0x05010400u);   // r0b0 r1b0 r0b1 r1b1
    const uint32_t t1 = __builtin_amdgcn_perm(r3, r2, 0x05010400u);   // r2b0 r3b0 r2b1 r3b1
    const uint32_t t2 = __builtin_amdgcn_perm(r1, r0, 0x07030602u);   // r0b2 r1b2 r0b3 r1b3
    const uint32_t t3 = __builtin_amdgcn_perm(r3, r2, 0x07030602u);
    col[0] = __builtin_amdgcn_perm(t1, t0, 0x05040100u);
    col[1] = __builtin_amdgcn_perm(t1, t0, 0x07060302u);
    col[2] = __builtin_amdgcn_perm(t3, t2, 0x05040100u);
    col[3] = __builtin_amdgcn_perm(t3, t2, 0x07060302u);
}

// ---------------------------------------------------------------------------
// Skinny GEMM over a [K,N] B in place, M <= 16 (A rows padded to 16):
// v_mfma_i32_16x16x64_i8 with each B fragment built by two transposed LDS
// reads (lds_read_tr8) from k rows staged as they lie in memory. A workgroup
// of 4 waves owns a group of 16 CB columns and one of sk.splits K ranges;
// wave w streams its own contiguous run of 64-row steps (16 CB bytes per
// row, whole cache lines, in 1 KiB DMA instructions) through an NSW-slot
// ring of its own, with the step's A fragments (16 bytes per lane, from L2)
// loaded beside it. The waves meet in LDS. With one K range the workgroup
// runs the output pass; with several it writes its int32 partials
// [split][M][N] (device-coherent sc1 stores), then its flag (the launch
// epoch), then reads every split's flag: a workgroup that finds them all set
// sums the column group's splits in split order and runs the output pass --
// the last to arrive always does, and one that reads the flags at the same
// moment writes the same bits -- then clears the flags, so a replayed graph
// (same epoch) finds them clear. No second launch.
// ---------------------------------------------------------------------------
template <int NSW, int CB>
__global__ __launch_bounds__(256) void gemv_i8_kn_tr(GemmI8Kern p, RingSplit sk, int groups)
{
    constexpr int CW = 16 * CB;             // columns per workgroup: CB blocks of 16
    constexpr int STEP = 64 * CW;           // bytes per 64-row step
    constexpr int Q = STEP / 1024;          // DMA instructions per step
    constexpr int RPQ = 1024 / CW;          // rows per DMA instruction
    constexpr int L = Q + 1;                // vector-memory ops per step: the DMA + 1 A load
    static_assert(CB == 8, "128-byte row segments (lds_tr8_ready ties 8 column blocks)");
    static_assert(NSW >= 1 && (NSW - 1) * L < 64, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) int8_t ring[4][NSW][STEP];
    static_assert(3 * CB * 64 * 16 <= 4 * NSW * STEP, "the waves' partial tiles fit the ring");
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int cg = blockIdx.x % groups, sp = blockIdx.x / groups;
    const int n0 = cg * CW;
    const int T = p.k / 64;
    const int s0 = (int)((int64_t)T * sp / sk.splits), s1 = (int)((int64_t)T * (sp + 1) / sk.splits);
    const int w0 = s0 + (s1 - s0) * wave / 4, w1 = s0 + (s1 - s0) * (wave + 1) / 4;
    const int nst = w1 - w0;

    // slot of 16-byte chunk c in k row r: the transposed reads of 32 lanes
    // (rows r0..r0+7 and r0+16..r0+23 of one chunk) fall in 16 distinct
    // 16-byte bank groups (128-byte rows: two rows per 256-byte bank row)
    auto swz = [](int r) {
        return CB == 8 ? ((((r >> 1) & 3) << 1) | ((r >> 4) & 1)) : (((r & 7) << 1) | ((r >> 4) & 1));
    };
    // the descriptor ends at B's last byte: chunks past column N of the last
    // row read 0 (earlier rows' read the next row: never stored)
    const BufRsrc rsb = buffer_rsrc(p.b + n0, (int)((int64_t)(p.k - 1) * p.ldb + (p.n - n0)));
    int b_off[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int r = q * RPQ + lane / CB;
        b_off[q] = r * (int)p.ldb + (((lane % CB) ^ swz(r)) << 4);
    }
    const int arow = lane & 15;
    const int8_t* a_row = p.a + (int64_t)min(arow, p.m - 1) * p.lda;
    const int kq = 16 * (lane >> 4);
    v4i fa[NSW];
    auto issue = [&](int st, int u) {
        int8_t* dst = ring[wave][u];
        fa[u] = *reinterpret_cast<const v4i*>(a_row + st * 64 + kq);
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            buffer_load_lds16<2>(rsb, dst + q * 1024, b_off[q], st * 64 * (int)p.ldb);
        }
    };
    // B fragment of column block cb (16 columns) from a staged step: lane
    // (group g, index i) reads k row 16 g + (i >> 1) (+8), columns 16 cb +
    // 8 (i & 1); lane l receives column 16 cb + (l & 15) at k 16 g + 0..15
    const int tr_k = 16 * (lane >> 4) + ((lane & 15) >> 1);
    const int tr_b = 8 * (lane & 1);
    v4i acc[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        acc[cb] = v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < NSW; ++u) {
        if (u < nst) {
            issue(w0 + u, u);
        }
    }
    for (int t = 0; t < nst; t += NSW) {
#pragma unroll
        for (int u = 0; u < NSW; ++u) {
            if (t + u < nst) {
                const int ahead = min(nst - 1 - (t + u), NSW - 1);
                if (ahead <= 0) {
                    wait_vmcnt<0>();
                } else if (NSW >= 2 && ahead == 1) {
                    wait_vmcnt<(NSW >= 2 ? L : 0)>();
                } else if (NSW >= 3 && ahead == 2) {
                    wait_vmcnt<(NSW >= 3 ? 2 * L : 0)>();
                } else {
                    wait_vmcnt<(NSW >= 4 ? 3 * L : 0)>();
                }
                asm volatile("" ::: "memory");
                const int8_t* st = ring[wave][u];
                v2i lo[CB], hi[CB];
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    // the column block is chunk cb of the staged row
                    const int k0 = tr_k;
                    lo[cb] = lds_read_tr8_asm(st + k0 * CW + ((cb ^ swz(k0)) << 4) + tr_b);
                    hi[cb] = lds_read_tr8_asm(st + (k0 + 8) * CW + ((cb ^ swz(k0 + 8)) << 4) + tr_b);
                }
                lds_tr8_ready(lo, hi);
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    acc[cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[u], v4i{lo[cb].x, lo[cb].y, hi[cb].x, hi[cb].y},
                                                                   acc[cb], 0, 0, 0);
                }
                // the slot's reads are done before the next step's DMA reuses it
                __builtin_amdgcn_s_waitcnt(0xc07f);
                asm volatile("" ::: "memory");
                if (t + u + NSW < nst) {
                    issue(w0 + t + u + NSW, u);
                }
            }
        }
    }
    __syncthreads();
    v4i* red = reinterpret_cast<v4i*>(&ring[0][0][0]);
    if (wave > 0) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            red[((wave - 1) * CB + cb) * 64 + lane] = acc[cb];
        }
    }
    __syncthreads();
    // 16x16 layout: lane holds column (lane & 15) of the block, rows 4 (lane >> 4) + r
    if (sk.splits == 1) {
        if (wave != 0) {
            return;
        }
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            const v4i v = acc[cb] + red[(0 * CB + cb) * 64 + lane] + red[(1 * CB + cb) * 64 + lane] +
                          red[(2 * CB + cb) * 64 + lane];
            const int n = n0 + 16 * cb + (lane & 15);
            if (n < p.n) {
                const EpiCol c = epi_col(p.ep, n);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = 4 * (lane >> 4) + r;
                    if (m < p.m) {
                        epi_store(p.ep, epi_row(p.ep, m), c, v[r],
                                  static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes, n);
                    }
                }
            }
        }
        return;
    }
    // the split's partials (byte offsets fit 32 bits: splits * M * N * 4 <
    // 2^31, checked by the plan), then its flag
    const BufRsrc rpart = buffer_rsrc(sk.part);
    const BufRsrc rflag = buffer_rsrc(sk.flag + (int64_t)cg * sk.splits);
    __shared__ int s_all;
    if (wave == 0) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            const v4i v = acc[cb] + red[(0 * CB + cb) * 64 + lane] + red[(1 * CB + cb) * 64 + lane] +
                          red[(2 * CB + cb) * 64 + lane];
            const int n = n0 + 16 * cb + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 4 * (lane >> 4) + r;
                if (n < p.n && m < p.m) {
                    buffer_store4_sc1(rpart, v[r], ((sp * p.m + m) * p.n + n) * 4);
                }
            }
        }
        wait_vmcnt<0>();
        if (lane == 0) {
            buffer_store8_sc1(rflag, sk.epoch, sp * 8);
        }
        wait_vmcnt<0>();
        bool all = true;
        for (int f0 = 0; f0 < sk.splits; f0 += 64) {
            const uint64_t f = f0 + lane < sk.splits ? buffer_load8_sc1(rflag, (f0 + lane) * 8) : sk.epoch;
            all = all && __builtin_amdgcn_ballot_w64(f != sk.epoch) == 0;
        }
        if (lane == 0) {
            s_all = all;
        }
    }
    __syncthreads();
    if (!s_all) {
        return;
    }
    // every split has published: 4 consecutive columns of one row per
    // thread, the splits summed in split order (exact: integers)
    const int q = threadIdx.x & (CW / 4 - 1);
    const int n = n0 + 4 * q;
    if (n < p.n) {
        const EpiCol c[4] = {epi_col(p.ep, n), epi_col(p.ep, n + 1), epi_col(p.ep, n + 2), epi_col(p.ep, n + 3)};
        const bool plain32 = p.ep.out_kind == NNOPS_OUT_S32 && !p.ep.compensate;
        for (int m = threadIdx.x / (CW / 4); m < p.m; m += 256 / (CW / 4)) {
            // four splits' loads in flight at a time
            v4i sum = v4i{0, 0, 0, 0};
            int sp2 = 0;
            for (; sp2 + 3 < sk.splits; sp2 += 4) {
                const int o = ((sp2 * p.m + m) * p.n + n) * 4, st = p.m * p.n * 4;
                const v4i x0 = buffer_load16_sc1(rpart, o), x1 = buffer_load16_sc1(rpart, o + st);
                const v4i x2 = buffer_load16_sc1(rpart, o + 2 * st), x3 = buffer_load16_sc1(rpart, o + 3 * st);
                sum += (x0 + x1) + (x2 + x3);
            }
            for (; sp2 < sk.splits; ++sp2) {
                sum += buffer_load16_sc1(rpart, ((sp2 * p.m + m) * p.n + n) * 4);
            }
            char* crow = static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes;
            if (plain32) {
                // an int32 destination without zero-point terms: bias and Relu
                const bool relu = p.ep.act == NNOPS_ACT_RELU;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int32_t v = sum[e] + c[e].bias;
                    reinterpret_cast<int32_t*>(crow)[n + e] = (relu && v < 0) ? 0 : v;
                }
                continue;
            }
            const EpiRow row = epi_row(p.ep, m);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                epi_store(p.ep, row, c[e], sum[e], crow, n + e);
            }
        }
    }
    for (int f = (int)threadIdx.x; f < sk.splits; f += (int)blockDim.x) {
        buffer_store8_sc1(rflag, 0ull, f * 8);
    }
}

template <int MT, int CPL, int W, int U>
__global__ __launch_bounds__(W * 64) void gemv_i8_kn(GemmI8Kern p, RingSplit sk, KnSplit ks)
{
    constexpr int D = CPL / 4;                   // dwords per lane per row
    // U k-quads per batch (4 U rows in flight); the waves' sums meet in one
    // LDS array through integer atomic adds (exact in any order)
    __shared__ int32_t red[MT * CPL][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    for (int i = threadIdx.x; i < MT * CPL * 64; i += W * 64) {
        (&red[0][0])[i] = 0;
    }
    const int chunk = blockIdx.x % ks.chunks;
    const int split = blockIdx.x / ks.chunks;
    const int n = chunk * 64 * CPL + lane * CPL;
    const bool live = n < p.n;
    // split s of S takes k-quads [s Q / S, (s + 1) Q / S) and its W waves
    // equal parts of that range, so any S fills the CUs evenly
    const int nquad = p.k / 4;
    const int qs0 = (int)((int64_t)split * nquad / sk.splits);
    const int qs1 = (int)((int64_t)(split + 1) * nquad / sk.splits);
    const int qw0 = qs0 + (int)((int64_t)wave * (qs1 - qs0) / W);
    const int qw1 = qs0 + (int)((int64_t)(wave + 1) * (qs1 - qs0) / W);

    int32_t acc[MT][CPL];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            acc[m][c] = 0;
        }
    }
    const int8_t* bcol = p.b + (live ? n : 0);
    for (int q = qw0; q < qw1; q += U) {
        const int nq = min(U, qw1 - q);       // wave-uniform
        const int k = 4 * q;
        uint32_t rows[4 * U][D];
#pragma unroll
        for (int r = 0; r < 4 * U; ++r) {
            const int8_t* src = bcol + (int64_t)(k + r) * p.ldb;
            if (r < 4 * nq) {
                if constexpr (D == 4) {
                    const v4i v = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(src));
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        rows[r][d] = (uint32_t)v[d];
                    }
                } else {
                    rows[r][0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(src));
                }
            } else {
#pragma unroll
                for (int d = 0; d < D; ++d) {
                    rows[r][d] = 0u;
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (u >= nq) {
                break;
            }
            int32_t aq[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const int mm = m < p.m ? m : 0;
                aq[m] = *reinterpret_cast<ScalarI32Ptr>((uintptr_t)(p.a + (int64_t)mm * p.lda + k + 4 * u));
            }
#pragma unroll
            for (int d = 0; d < D; ++d) {
                uint32_t col[4];
                transpose4x4_bytes(rows[4 * u][d], rows[4 * u + 1][d], rows[4 * u + 2][d], rows[4 * u + 3][d], col);
#pragma unroll
                for (int m = 0; m < MT; ++m) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        acc[m][4 * d + c] = __builtin_amdgcn_sdot4(aq[m], (int)col[c], acc[m][4 * d + c], false);
                    }
                }
            }
        }
    }
    __syncthreads();   // red is cleared
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            if (m < p.m) {
                atomicAdd(&red[m * CPL + c][lane], acc[m][c]);
            }
        }
    }
    __syncthreads();
    // Thread t takes chunk column r = t % (64 CPL) (lane r / CPL, element
    // r % CPL) of row t / (64 CPL), so consecutive threads store consecutive
    // int32 partials.
    const int nc0 = chunk * 64 * CPL;
    int32_t* part = sk.part + (int64_t)split * p.m * p.n;
    for (int idx = threadIdx.x; idx < MT * CPL * 64; idx += W * 64) {
        const int m = idx / (CPL * 64);
        const int r = idx % (CPL * 64);
        if (m < p.m && nc0 + r < p.n) {
            part[(int64_t)m * p.n + nc0 + r] = red[m * CPL + r % CPL][r / CPL];
        }
    }
}

// ---------------------------------------------------------------------------
// Prepasses
// ---------------------------------------------------------------------------
// dst[c][r] = src[r][c] for r < R, c < C; dst columns r in [R, Rp) are zeroed.
// The same transpose in 256-row x 64-column tiles with 16-byte accesses on
// both sides (source rows, pitch, destination and its pitch 16-byte aligned,
// Rp % 16 == 0): each thread loads four 16-byte row pieces into LDS (row
// pitch 17 dwords), then reads a 16-row x 4-column block as 16 dwords,
// transposes it in registers (v_perm, 4 x 4 bytes at a time) and stores four
// 16-byte destination pieces (the byte-wise kernel below, kept for unaligned
// operands, moves one byte per load and store).
__global__ __launch_bounds__(256) void transpose_i8_v(const int8_t* src, int64_t lds_, int R, int C,
                                                      int8_t* dst, int64_t ldd, int Rp)
{
    constexpr int TR = 256, TC = 64, P = TC / 4 + 1;   // rows, columns, LDS pitch in dwords
    __shared__ uint32_t tile[TR * P];
    const int r0 = blockIdx.y * TR;
    const int c0 = blockIdx.x * TC;
    const int t = threadIdx.x;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int idx = q * 256 + t;
        const int row = idx >> 2, seg = idx & 3;
        const int r = r0 + row, c = c0 + 16 * seg;
        v4i v = v4i{0, 0, 0, 0};
        if (r < R && c < C) {
            const int8_t* sp = src + (int64_t)r * lds_ + c;
            if (c + 16 <= C) {
                v = *reinterpret_cast<const v4i*>(sp);
            } else {
                uint32_t w[4] = {0u, 0u, 0u, 0u};
                for (int b = 0; b < C - c; ++b) {
                    w[b >> 2] |= (uint32_t)(uint8_t)sp[b] << (8 * (b & 3));
                }
                v = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
            }
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            tile[row * P + 4 * seg + d] = (uint32_t)v[d];
        }
    }
    __syncthreads();
    const int c4 = t & 15, r16 = t >> 4;
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        w[i] = tile[(16 * r16 + i) * P + c4];
    }
    uint32_t col[4][4];   // [column j][row quad g]
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        uint32_t cq[4];
        transpose4x4_bytes(w[4 * g], w[4 * g + 1], w[4 * g + 2], w[4 * g + 3], cq);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            col[j][g] = cq[j];
        }
    }
    const int r = r0 + 16 * r16;
    if (r >= Rp) {
        return;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = c0 + 4 * c4 + j;
        if (c < C) {
            *reinterpret_cast<v4i*>(dst + (int64_t)c * ldd + r) =
                v4i{(int)col[j][0], (int)col[j][1], (int)col[j][2], (int)col[j][3]};
        }
    }
}

__global__ __launch_bounds__(256) void transpose_i8(const int8_t* src, int64_t lds_, int R, int C,
                                                   int8_t* dst, int64_t ldd, int Rp)
{
    __shared__ int8_t tile[64][65];
    const int r0 = blockIdx.y * 64;
    const int c0 = blockIdx.x * 64;
    const int tx = threadIdx.x & 63;
    const int ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        const int r = r0 + i, c = c0 + tx;
        tile[i][tx] = (r < R && c < C) ? src[(int64_t)r * lds_ + c] : (int8_t)0;
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int c = c0 + i, r = r0 + tx;
        if (c < C && r < Rp) {
            dst[(int64_t)c * ldd + r] = tile[tx][i];
        }
    }
}

// dst[c][r] = src[r][c] (r < R, c < C; columns r in [R, Rp) zeroed): the
// 16-byte tiled kernel where its alignment holds, else the byte-wise one.
void launch_transpose_i8(const int8_t* src, int64_t lds_, int R, int C, int8_t* dst, int64_t ldd, int Rp,
                         hipStream_t s)
{
    if (((uintptr_t)src % 16) == 0 && lds_ % 16 == 0 && ((uintptr_t)dst % 16) == 0 && ldd % 16 == 0 &&
        Rp % 16 == 0) {
        const dim3 grid((unsigned)((C + 63) / 64), (unsigned)((Rp + 255) / 256));
        NNOPS_LAUNCH(transpose_i8_v, grid, dim3(256), 0, s, src, lds_, R, C, dst, ldd, Rp);
    } else {
        const dim3 grid((unsigned)((C + 63) / 64), (unsigned)((Rp + 63) / 64));
        NNOPS_LAUNCH(transpose_i8, grid, dim3(256), 0, s, src, lds_, R, C, dst, ldd, Rp);
    }
}

// The same for 2-byte elements (an f16 [K][N] B staged as [N][Kp]).
__global__ __launch_bounds__(256) void transpose_b16(const uint16_t* src, int64_t lds_, int R, int C,
                                                    uint16_t* dst, int64_t ldd, int Rp)
{
    __shared__ uint16_t tile[64][65];
    const int r0 = blockIdx.y * 64;
    const int c0 = blockIdx.x * 64;
    const int tx = threadIdx.x & 63;
    const int ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        const int r = r0 + i, c = c0 + tx;
        tile[i][tx] = (r < R && c < C) ? src[(int64_t)r * lds_ + c] : (uint16_t)0;
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int c = c0 + i, r = r0 + tx;
        if (c < C && r < Rp) {
            dst[(int64_t)c * ldd + r] = tile[tx][i];
        }
    }
}

// out[r] = sum_k row r (u8 reads unsigned). One wave per row.
__global__ __launch_bounds__(256) void rowsum_i8(const int8_t* src, int64_t ld, int R, int K, int u8,
                                                int32_t* out)
{
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= R) {
        return;
    }
    const int8_t* row = src + (int64_t)r * ld;
    int32_t s = 0;
    for (int k = lane; k < K; k += 64) {
        s += u8 ? (int32_t)(uint8_t)row[k] : (int32_t)row[k];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        s += __shfl_xor(s, off, 64);
    }
    if (lane == 0) {
        out[r] = s;
    }
}

// Row copy into a wider, zero-padded pitch (the prepack of an [N,K] B):
// 16 bytes per thread where source and destination allow it.
__global__ __launch_bounds__(256) void pad_rows_i8(const int8_t* src, int64_t lds_, int R, int C,
                                                  int8_t* dst, int64_t ldd)
{
    const int64_t chunks = ldd / 16;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= (int64_t)R * chunks) {
        return;
    }
    const int r = (int)(t / chunks);
    const int c0 = (int)(t - (int64_t)r * chunks) * 16;
    const int8_t* s = src + (int64_t)r * lds_;
    int8_t v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        v[i] = c0 + i < C ? s[c0 + i] : (int8_t)0;
    }
    int4 o;
    __builtin_memcpy(&o, v, 16);
    *reinterpret_cast<int4*>(dst + (int64_t)r * ldd + c0) = o;
}

// ---------------------------------------------------------------------------
// Host side: workspace plan and dispatch.
// ---------------------------------------------------------------------------
constexpr size_t kAlign = 256;
inline size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }
inline int64_t round16(int64_t x) { return (x + 15) / 16 * 16; }

// Which ring-kernel configuration a call takes (all zero: another kernel).
struct RingPlan {
    int bm = 0, bn = 0;     // block tile
    int bk = 64;            // k bytes per staged row (128 when K allows)
    int splits = 0;         // K splits (1: no split)
    int mode = -1;          // RING_S8 / RING_S32 / RING_PART
    bool trb = false;       // B is [K,N] row-major, read in place (TRB)
};

// Column GEMV plan ([K,N] B consumed in place, M <= 16).
struct KnPlan {
    int cpl = 0;            // columns per lane (0: not taken)
    int w = 0;              // waves per workgroup
    int chunks = 0, splits = 0;
    bool tr = false;        // gemv_i8_kn_tr (chunks: its 128-column groups)
};

inline int kn_mt(int64_t m) { return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : m <= 8 ? 8 : 16; }

struct WsPlan {
    size_t r_a = 0, r_b = 0, a_t = 0, b_t = 0, part = 0, flag = 0, total = 0;
    int64_t kp = 0;
    RingPlan ring;
    KnPlan kn;
};

inline bool aligned16(const void* p, int64_t ld) { return ((uintptr_t)p % 16 == 0) && (ld % 16 == 0); }

// M <= 16 with a [K,N] B: 16-byte (M <= 2) or 4-byte column groups per lane,
// K % 16 == 0, dword-aligned A rows (scalar loads), no term that needs the
// column sums of B (u8 A, A zero points). About 512 workgroups of 8 (or 4)
// waves, row ranges a multiple of 16.
KnPlan plan_kn(const NnopsGemmI8Args& g)
{
    KnPlan r;
    if (g.trans_b || g.trans_a || g.m > 16 || g.k % 16 != 0 || g.a_u8 || g.zp_a != nullptr || g.zp_a_scalar != 0) {
        return r;
    }
    // (8 columns per lane with 32 rows in flight measured slower for
    // 4 <= M <= 16: 17.1 / 32.1 us against 14.8 / 28.3 at M = 4 / 16)
    // 3 <= M <= 16, 64-row steps, 16-byte rows: the transposed-read MFMA
    // kernel, K split so about two workgroups per CU stream at once
    // (measured at config 3, N = 11008, call totals with the reduce: 128-byte
    // row segments and ~512 workgroups 15.2 / 16.6 us at M = 4 / 16; 256-byte
    // segments 18.7 / 20.0 (256 workgroups) and 21.8 / 27.0 (512); no K split
    // (86 workgroups) 37.8 / 38.5; at M = 1..2 the column GEMV stays faster,
    // 13.8 against 14.9 us). With the splits meeting in the launch: 14.6 /
    // 16.5 us at 5 splits, the same at 4, 16.6 / 18.8 at 3, 19.7 / 21.8 at 6
    // (516 workgroups: a second round), 17.3 / 18.8 at 8.
    if (g.m >= 3 && g.k % 64 == 0 && g.n % 4 == 0 && aligned16(g.b, g.ldb) &&
        aligned16(static_cast<const int8_t*>(g.a), g.lda) && g.k * g.ldb + g.n < (int64_t)INT32_MAX) {
        r.tr = true;
        r.cpl = 8;          // column blocks of 16 per workgroup
        r.w = 4;
        r.chunks = (int)((g.n + 127) / 128);
        r.splits = (int)std::max<int64_t>(1, std::min<int64_t>(512 / r.chunks, g.k / 64 / 4));
        if ((int64_t)r.splits * g.m * g.n * 4 >= INT32_MAX) {
            return KnPlan{};
        }
        return r;
    }
    const int cpl = 4;
    if (g.n % cpl != 0 || g.n % 4 != 0 || ((uintptr_t)g.b % cpl) != 0 || (g.ldb % cpl) != 0 ||
        ((uintptr_t)g.a % 4) != 0 || (g.lda % 4) != 0) {
        return r;
    }
    const int mt = kn_mt(g.m);
    r.cpl = cpl;
    r.chunks = (int)((g.n + 64 * cpl - 1) / (64 * cpl));
    // 256-column chunks (4 columns per lane: every wave load is 256 bytes of
    // one row, two whole lines). K is split so the workgroups fill the CUs
    // about twice, each split at least 16 rows per wave. (Config 3, M = 1:
    // 43 chunks x 11 splits, 13.0 us per call; 1024-column chunks of 16-byte
    // lanes, 11 chunks x 23 splits of 16 waves, ran 13.6 at M = 1 and 15.1
    // against 13.5 at M = 2.)
    r.w = (mt * cpl >= 64) ? 4 : 8;
    const int per_cu = 2;
    const int64_t max_splits = std::max<int64_t>(1, g.k / (16 * r.w));
    r.splits = (int)std::min<int64_t>(max_splits, std::max(1, 256 * per_cu / r.chunks));
    if ((int64_t)r.splits * g.m * g.n * 4 >= INT32_MAX) {
        return KnPlan{};    // the partials' 32-bit buffer offsets
    }
    return r;
}


// The ring kernel needs 64-byte k steps, 16-byte-aligned k-contiguous rows,
// N % 4 == 0 (int32 groups), and 32-bit buffer offsets within a row panel.
// Tile shape by M: a 257..384-row problem takes two 192x128 tiles (384x128 when
// K % 128 != 0), 128x256 and 256x128 the small ones, 256x256 the rest. K is split when the
// tiles alone do not fill the 256 CUs (at least 8 k steps per split). The
// fused output modes need row-uniform parameters, no zero-point terms,
// half-away rounding, 16-byte-aligned tables and destination, and no split;
// everything else writes raw partials and runs gemm_i8_reduce.
// trb: B is the caller's [K,N] (row pitch ldb), read in place (its whole
// span within 32-bit buffer offsets). small_tiles: grids of fewer than 32
// tiles take 64 x 64 tiles of 4 waves instead (config 1, 128 x 1024 x 1024:
// 32 workgroups in place of 4).
RingPlan plan_ring(const NnopsGemmI8Args& g, const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                   bool trb = false, bool small_tiles = false)
{
    RingPlan r;
    if (g.m <= 16 || g.k % 64 != 0 || g.n % 4 != 0 || g.m < 64 || !aligned16(a, lda) || !aligned16(b, ldb)) {
        return r;
    }
    if (trb && (g.k * ldb + g.n >= (int64_t)INT32_MAX || ldb < g.n)) {
        return r;
    }
    r.trb = trb;
    if (g.m > 256 && g.m <= 384 && g.k % 128 == 0) {
        // two 192-row tiles: twice the tiles of one 384-row tile, so half the
        // K splits (and half the partial-sum traffic) fill the CUs
        r.bm = 192; r.bn = 128;
    } else if (g.m > 256 && g.m <= 384) {
        r.bm = 384; r.bn = 128;
    } else if (g.m <= 128) {
        r.bm = 128; r.bn = 256;
    } else if (g.m <= 256) {
        r.bm = 256; r.bn = 128;
    } else {
        r.bm = 256; r.bn = 256;
    }
    if (small_tiles && ((g.m + r.bm - 1) / r.bm) * ((g.n + r.bn - 1) / r.bn) < 32) {
        r.bm = 64; r.bn = 64;
    }
    if ((int64_t)r.bm * lda >= (int64_t)INT32_MAX || (!trb && (int64_t)r.bn * ldb >= (int64_t)INT32_MAX)) {
        r = RingPlan{};
        return r;
    }
    const int64_t tiles = ((g.m + r.bm - 1) / r.bm) * ((g.n + r.bn - 1) / r.bn);
    r.bk = (g.k % 128 == 0) ? 128 : 64;
    const int kt = (int)(g.k / r.bk);
    // at least 512 k per split, and no split below 16 k steps: a short ring
    // gains less from splitting than the reduce launch costs (config 1,
    // 128x1024x1024 s32: 10.5 + 3.9 us in two splits, 12.4 us unsplit)
    r.splits = kt < 16 ? 1 : (int)std::max<int64_t>(1, std::min<int64_t>(256 / tiles, kt / (512 / r.bk)));
    // (the 64 x 64 tiles of config 1 split 4 ways: 4.2 us ring + 3.4 us
    // reduce against 6.4 us unsplit)
    const bool compensate = g.a_u8 || g.zp_a != nullptr || g.zp_a_scalar != 0 || g.zp_b != nullptr ||
                            g.zp_b_scalar != 0;
    const bool tables16 = ((uintptr_t)g.bias % 16 == 0) && ((uintptr_t)g.s_b % 16 == 0);
    const bool fp_out = g.out_kind == NNOPS_OUT_F32 || g.out_kind == NNOPS_OUT_F16;
    const bool plain = !compensate && g.s_out_rows == nullptr && g.zp_out_rows == nullptr && !g.float_ep &&
                       !g.round_even && !fp_out && tables16 && ((uintptr_t)g.c % 16 == 0);
    r.mode = RING_PART;
    const size_t ebytes = g.out_kind == NNOPS_OUT_F16 ? 2 : 4;
    if (r.splits == 1 && fp_out && !compensate && (g.act == NNOPS_ACT_NONE || g.act == NNOPS_ACT_RELU) &&
        (uintptr_t)g.c % 16 == 0 && (g.ldc * ebytes) % 16 == 0 &&
        ((uintptr_t)g.s_b % 16) == 0 && (g.bias_fp == nullptr || (uintptr_t)g.bias_fp % (4 * ebytes) == 0)) {
        r.mode = RING_FP;      // dequantizing output pass fused
    } else if (r.splits == 1 && plain) {
        if (g.out_kind == NNOPS_OUT_S32 && (g.ldc * 4) % 16 == 0) {
            r.mode = RING_S32;
        } else if (g.out_kind != NNOPS_OUT_S32 && g.s_a == nullptr && g.ldc % 16 == 0 && g.n % 16 == 0) {
            r.mode = RING_S8;
        }
    }
    return r;
}

WsPlan plan_workspace(const NnopsGemmI8Args& g)
{
    WsPlan w;
    size_t off = 0;
    w.kp = round16(g.k);
    w.r_a = off; off += align_up((size_t)g.m * 4);
    w.r_b = off; off += align_up((size_t)g.n * 4);
    const int8_t* a = static_cast<const int8_t*>(g.a);
    const int8_t* b = g.b;
    int64_t lda = g.lda, ldb = g.ldb;
    if (g.trans_a) {
        w.a_t = off; off += align_up((size_t)g.m * (size_t)w.kp);
        a = nullptr;      // staged copies are 256-byte aligned with a 16-byte pitch
        lda = w.kp;
    }
    w.kn = plan_kn(g);
    if (w.kn.cpl != 0) {
        w.part = off; off += align_up((size_t)w.kn.splits * (size_t)g.m * (size_t)g.n * 4);
        if (w.kn.tr && w.kn.splits > 1) {
            // the splits' completion flags (gemv_i8_kn_tr meets them in the launch)
            w.flag = off; off += align_up((size_t)w.kn.chunks * (size_t)w.kn.splits * 8);
        }
        w.total = off;
        return w;
    }
    // a [K,N] B goes to the ring in place when it takes it and no column
    // sums of B are needed (they are summed over the staged copy's rows)
    const bool need_rb = g.a_u8 || g.zp_a != nullptr || g.zp_a_scalar != 0;
    if (!g.trans_b && !need_rb) {
        w.ring = plan_ring(g, a, lda, b, ldb, true, true);
    }
    if (!g.trans_b && w.ring.mode < 0) {
        w.b_t = off; off += align_up((size_t)g.n * (size_t)w.kp);
        b = nullptr;
        ldb = w.kp;
    }
    if (!w.ring.trb) {
        w.ring = plan_ring(g, a, lda, b, ldb, false, true);
    }
    if (w.ring.mode == RING_PART) {
        w.part = off; off += align_up((size_t)w.ring.splits * (size_t)g.m * (size_t)g.n * 4);
    }
    w.total = off;
    return w;
}

template <int BM, int BN, int WM, int WN, int WPE, bool FULLK, bool ALIGNED>
void launch_gemm_epi(const GemmI8Kern& k, int epi, hipStream_t s)
{
    const int tiles = ((k.m + BM - 1) / BM) * ((k.n + BN - 1) / BN);
    const dim3 grid(tiles), block(WM * WN * 64);
    if (k.a_xor != 0u) {
        NNOPS_LAUNCH((gemm_i8_mfma<BM, BN, WM, WN, WPE, FULLK, ALIGNED, true, EPI_GENERIC>), grid, block, 0, s, k);
    } else if (epi == EPI_S8) {
        NNOPS_LAUNCH((gemm_i8_mfma<BM, BN, WM, WN, WPE, FULLK, ALIGNED, false, EPI_S8>), grid, block, 0, s, k);
    } else if (epi == EPI_S32) {
        NNOPS_LAUNCH((gemm_i8_mfma<BM, BN, WM, WN, WPE, FULLK, ALIGNED, false, EPI_S32>), grid, block, 0, s, k);
    } else {
        NNOPS_LAUNCH((gemm_i8_mfma<BM, BN, WM, WN, WPE, FULLK, ALIGNED, false, EPI_GENERIC>), grid, block, 0, s, k);
    }
}

template <int BM, int BN, int WM, int WN, int WPE>
void launch_gemm(const GemmI8Kern& k, bool aligned, bool fullk, int epi, hipStream_t s)
{
    if (fullk) {
        launch_gemm_epi<BM, BN, WM, WN, WPE, true, true>(k, epi, s);
    } else if (aligned) {
        launch_gemm_epi<BM, BN, WM, WN, WPE, false, true>(k, epi, s);
    } else {
        launch_gemm_epi<BM, BN, WM, WN, WPE, false, false>(k, epi, s);
    }
}

template <int BM, int BN, int WM, int WN, int BK, int NS, bool F16 = false>
void launch_ring_bk(const GemmI8Kern& k, const RingSplit& sk, int mode, bool flip, bool trb, hipStream_t s)
{
    const unsigned blocks = (unsigned)(((k.m + BM - 1) / BM) * ((k.n + BN - 1) / BN) * sk.splits);
    const dim3 block(WM * WN * 64);
    if (trb) {
        // [K,N] B in place; plain A (no u8 flip: its column sums need the copy)
        if constexpr (!F16) {
            if (mode == RING_S8) {
                NNOPS_LAUNCH((gemm_i8_ring<BM, BN, WM, WN, BK, NS, RING_S8, false, false, true>), dim3(blocks), block,
                             0, s, k, sk);
            } else if (mode == RING_S32) {
                NNOPS_LAUNCH((gemm_i8_ring<BM, BN, WM, WN, BK, NS, RING_S32, false, false, true>), dim3(blocks),
                             block, 0, s, k, sk);
            } else if (mode == RING_FP) {
                NNOPS_LAUNCH((gemm_i8_ring<BM, BN, WM, WN, BK, NS, RING_FP, false, false, true>), dim3(blocks), block,
                             0, s, k, sk);
            } else {
                NNOPS_LAUNCH((gemm_i8_ring<BM, BN, WM, WN, BK, NS, RING_PART, false, false, true>), dim3(blocks),
                             block, 0, s, k, sk);
            }
        }
        return;
    }
    if constexpr (F16) {
        (void)flip;
        if (mode == RING_FP) {
            NNOPS_LAUNCH((gemm_i8_ring<BM, BN, WM, WN, BK, NS, RING_FP, false, true>), dim3(blocks), block, 0,
                               s, k, sk);
        } else {
            NNOPS_LAUNCH((gemm_i8_ring<BM, BN, WM, WN, BK, NS, RING_PART, false, true>), dim3(blocks), block,
                               0, s, k, sk);
        }
        return;
    }
    if (flip) {
        NNOPS_LAUNCH((gemm_i8_ring<BM, BN, WM, WN, BK, NS, RING_PART, true>), dim3(blocks), block, 0, s, k, sk);
    } else if (mode == RING_S8) {
        NNOPS_LAUNCH((gemm_i8_ring<BM, BN, WM, WN, BK, NS, RING_S8, false>), dim3(blocks), block, 0, s, k, sk);
    } else if (mode == RING_S32) {
        NNOPS_LAUNCH((gemm_i8_ring<BM, BN, WM, WN, BK, NS, RING_S32, false>), dim3(blocks), block, 0, s, k, sk);
    } else if (mode == RING_FP) {
        NNOPS_LAUNCH((gemm_i8_ring<BM, BN, WM, WN, BK, NS, RING_FP, false>), dim3(blocks), block, 0, s, k, sk);
    } else {
        NNOPS_LAUNCH((gemm_i8_ring<BM, BN, WM, WN, BK, NS, RING_PART, false>), dim3(blocks), block, 0, s, k, sk);
    }
}

// 128-byte staged rows (whole cache lines: twice the bytes per L2 request of
// 64-byte rows, which is what limits a CU's load rate) in 2 slots when K
// allows, else 64-byte rows in 4 slots.
template <int BM, int BN, int WM, int WN, bool F16 = false>
void launch_ring_cfg(const GemmI8Kern& k, const RingSplit& sk, int bk, int mode, bool flip, bool trb, hipStream_t s)
{
    if (bk == 128) {
        // three stage slots where the LDS holds them (config 5's 192x128 tiles:
        // 33.7 -> 32.9 us), two for the 256x256 tile; the 64 x 64 tiles of
        // small grids keep 8 stages in flight (their latency is the call's)
        if constexpr (BM + BN <= 128) {
            launch_ring_bk<BM, BN, WM, WN, 128, 8, F16>(k, sk, mode, flip, trb, s);
        } else if constexpr ((BM + BN) * 128 * 3 <= 160 * 1024 && BM + BN < 512) {
            launch_ring_bk<BM, BN, WM, WN, 128, 3, F16>(k, sk, mode, flip, trb, s);
        } else {
            launch_ring_bk<BM, BN, WM, WN, 128, 2, F16>(k, sk, mode, flip, trb, s);
        }
    } else if constexpr (BM % (16 * WM * WN) == 0 && BN % (16 * WM * WN) == 0) {
        launch_ring_bk<BM, BN, WM, WN, 64, 4, F16>(k, sk, mode, flip, trb, s);
    }
}

template <int MT>
void launch_kn_mt(const GemmI8Kern& k, const RingSplit& sk, const KnSplit& ks, int cpl, int w, hipStream_t s)
{
    const dim3 grid((unsigned)(ks.chunks * sk.splits));
    (void)cpl;                              // the plan takes 4 columns per lane
    if (w == 4) {
        NNOPS_LAUNCH((gemv_i8_kn<MT, 4, 4, 4>), grid, dim3(256), 0, s, k, sk, ks);
    } else {
        NNOPS_LAUNCH((gemv_i8_kn<MT, 4, 8, 4>), grid, dim3(512), 0, s, k, sk, ks);
    }
}

// gemm_i8_reduce_q's conditions: an s8 / u8 destination with row-uniform
// parameters and no zero-point terms, 16-byte-aligned tables and 4-byte
// aligned destination rows, an identity / Relu / GELU activation (GELU only
// with the float epilogue).
bool reduce_q_ok(const GemmI8Kern& k)
{
    const EpiParams& e = k.ep;
    return (e.out_kind == NNOPS_OUT_S8 || e.out_kind == NNOPS_OUT_U8) && !e.compensate && e.s_a == nullptr &&
           e.s_out_rows == nullptr && e.zp_out_rows == nullptr && ((uintptr_t)e.s_b % 16) == 0 &&
           ((uintptr_t)e.bias % 16) == 0 && ((uintptr_t)k.c % 4) == 0 && (k.ldc_bytes % 4) == 0 &&
           (e.act == NNOPS_ACT_NONE || e.act == NNOPS_ACT_RELU || (e.act == NNOPS_ACT_GELU && e.float_ep));
}

template <int ACT>
void launch_reduce_q_act(const GemmI8Kern& k, const RingSplit& sk, const dim3& grid, hipStream_t s)
{
    const EpiParams& e = k.ep;
    if (!e.float_ep) {
        if constexpr (ACT != NNOPS_ACT_GELU) {
            NNOPS_LAUNCH((gemm_i8_reduce_q<ACT, false, false, false>), grid, dim3(256), 0, s, k, sk);
        }
    } else if (!e.add_to) {
        NNOPS_LAUNCH((gemm_i8_reduce_q<ACT, true, false, false>), grid, dim3(256), 0, s, k, sk);
    } else if (e.residual_pre) {
        NNOPS_LAUNCH((gemm_i8_reduce_q<ACT, true, true, true>), grid, dim3(256), 0, s, k, sk);
    } else {
        NNOPS_LAUNCH((gemm_i8_reduce_q<ACT, true, true, false>), grid, dim3(256), 0, s, k, sk);
    }
}

void launch_reduce(const GemmI8Kern& k, const RingSplit& sk, hipStream_t s)
{
    const int64_t groups = (int64_t)k.m * (k.n / 4);
    if (sk.splits <= 8 && reduce_q_ok(k)) {
        const dim3 grid((unsigned)((k.n / 4 + 255) / 256), (unsigned)std::min<int64_t>(k.m, 65535));
        RingSplit q = sk;
        q.row_k = k.ep.s_a_scalar / k.ep.s_out;
        q.inv_out = 1.0f / k.ep.s_out;
        if (k.ep.act == NNOPS_ACT_GELU) {
            launch_reduce_q_act<NNOPS_ACT_GELU>(k, q, grid, s);
        } else if (k.ep.act == NNOPS_ACT_RELU) {
            launch_reduce_q_act<NNOPS_ACT_RELU>(k, q, grid, s);
        } else {
            launch_reduce_q_act<NNOPS_ACT_NONE>(k, q, grid, s);
        }
        return;
    }
    if (sk.splits > 8) {
        NNOPS_LAUNCH(gemm_i8_reduce<16>, dim3((unsigned)((groups * 16 + 255) / 256)), dim3(256), 0, s, k, sk);
    } else {
        NNOPS_LAUNCH(gemm_i8_reduce<1>, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, s, k, sk);
    }
}

void launch_kn(const GemmI8Kern& k, const KnPlan& r, int32_t* part, uint64_t* flag, hipStream_t s)
{
    RingSplit sk{};
    sk.splits = r.splits;
    sk.kt_per = 0;
    sk.part = part;
    if (r.tr) {
        sk.flag = flag;
        sk.epoch = next_launch_epoch();
        NNOPS_LAUNCH((gemv_i8_kn_tr<2, 8>), dim3((unsigned)(r.chunks * r.splits)), dim3(256), 0, s, k, sk,
                     r.chunks);
        return;
    }
    KnSplit ks;
    ks.chunks = r.chunks;
    switch (k.m) {
    case 1: launch_kn_mt<1>(k, sk, ks, r.cpl, r.w, s); break;
    case 2: launch_kn_mt<2>(k, sk, ks, r.cpl, r.w, s); break;
    case 3: case 4: launch_kn_mt<4>(k, sk, ks, r.cpl, r.w, s); break;
    case 5: case 6: case 7: case 8: launch_kn_mt<8>(k, sk, ks, r.cpl, r.w, s); break;
    default: launch_kn_mt<16>(k, sk, ks, r.cpl, r.w, s); break;
    }
    launch_reduce(k, sk, s);
}

// C = alpha * (the f16 ring's f32 partials summed in split order)
__global__ __launch_bounds__(256) void ring_f16_reduce(GemmI8Kern p, RingSplit sk)
{
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)p.m * p.n) {
        return;
    }
    const int64_t slab = (int64_t)p.m * p.n;
    float v = 0.0f;
    for (int sp = 0; sp < sk.splits; ++sp) {
        v += __builtin_bit_cast(float, sk.part[sp * slab + i]);
    }
    v = __fmul_rn(v, p.ep.s_a_scalar);
    const int m = (int)(i / p.n);
    const int n = (int)(i - (int64_t)m * p.n);
    char* crow = static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes;
    if (p.ep.out_kind == NNOPS_OUT_F16) {
        reinterpret_cast<_Float16*>(crow)[n] = (_Float16)v;
    } else {
        reinterpret_cast<float*>(crow)[n] = v;
    }
}

template <bool F16 = false>
void launch_ring(const GemmI8Kern& k, const RingPlan& r, int32_t* part, hipStream_t s)
{
    RingSplit sk;
    sk.splits = r.splits;
    sk.kt_per = (k.k / r.bk) / r.splits;
    sk.part = part;
    const bool flip = k.a_xor != 0u;
    if (r.bm == 384) {
        launch_ring_cfg<384, 128, 4, 2, F16>(k, sk, r.bk, r.mode, flip, r.trb, s);
    } else if (r.bm == 192) {
        launch_ring_cfg<192, 128, 2, 4, F16>(k, sk, r.bk, r.mode, flip, r.trb, s);
    } else if (r.bm == 128) {
        launch_ring_cfg<128, 256, 2, 4, F16>(k, sk, r.bk, r.mode, flip, r.trb, s);
    } else if (r.bm == 64) {
        if constexpr (!F16) {
            launch_ring_cfg<64, 64, 2, 2>(k, sk, r.bk, r.mode, flip, r.trb, s);
        }
    } else if (r.bn == 128) {
        launch_ring_cfg<256, 128, 4, 2, F16>(k, sk, r.bk, r.mode, flip, r.trb, s);
    } else {
        launch_ring_cfg<256, 256, 2, 4, F16>(k, sk, r.bk, r.mode, flip, r.trb, s);
    }
    if (r.mode == RING_PART) {
        if constexpr (F16) {
            NNOPS_LAUNCH(ring_f16_reduce, dim3((unsigned)(((int64_t)k.m * k.n + 255) / 256)), dim3(256), 0, s,
                               k, sk);
        } else {
            launch_reduce(k, sk, s);
        }
    }
}

// Which output-pass specialisation a call can take: the fast modes need
// row-uniform parameters, no zero-point terms, half-away rounding, and a
// destination that takes packed stores for every 4-column group.
int choose_epi(const NnopsGemmI8Args& g, const EpiParams& e)
{
    if (e.compensate || g.s_out_rows != nullptr || g.zp_out_rows != nullptr || g.float_ep ||
        g.round_even || (g.n % 4) != 0 || ((uintptr_t)g.c & 15) != 0 || epi_is_fp(e)) {
        return EPI_GENERIC;
    }
    if (g.out_kind == NNOPS_OUT_S32) {
        return (g.ldc * 4) % 16 == 0 ? EPI_S32 : EPI_GENERIC;
    }
    return (g.s_a == nullptr && g.ldc % 4 == 0) ? EPI_S8 : EPI_GENERIC;
}

}  // namespace
}  // namespace nnops_amd

using namespace nnops_amd;

namespace {
int64_t prepack_pitch(int64_t k) { return (k + 127) / 128 * 128; }

// The LDS skinny GEMM: M 5..16 (M <= 4 streams faster through the row GEMV),
// a block's 16 rows within a 32-bit buffer range.
bool gemv_lds_ok(const NnopsGemmI8Args& g)
{
    return g.m > 4 && (int64_t)16 * g.ldb + g.k < (int64_t)INT32_MAX;
}
}  // namespace

extern "C" size_t nnops_hip_prepack_i8_bytes(int64_t k, int64_t n)
{
    if (k < 0 || n < 0) {
        return 0;
    }
    return align_up((size_t)n * (size_t)prepack_pitch(k)) + (size_t)n * 4;
}

extern "C" int nnops_hip_prepack_i8(const int8_t* b, int64_t k, int64_t n, int64_t ldb, int32_t trans_b,
                                    void* out, void* stream)
{
    const TimingDisarm disarm;
    if (k < 0 || n < 0 || k > INT32_MAX || n > INT32_MAX) {
        return NNOPS_INVALID_ARGUMENT;
    }
    if (k == 0 || n == 0) {
        return NNOPS_OK;
    }
    if (b == nullptr || out == nullptr || (uintptr_t)out % 256 != 0 || ldb < (trans_b ? k : n)) {
        return NNOPS_INVALID_ARGUMENT;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t kp = prepack_pitch(k);
    int8_t* rows = static_cast<int8_t*>(out);
    int32_t* sums = reinterpret_cast<int32_t*>(static_cast<char*>(out) + align_up((size_t)n * (size_t)kp));
    if (trans_b) {
        const int64_t threads = n * (kp / 16);
        NNOPS_LAUNCH(pad_rows_i8, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, b, ldb, (int)n,
                           (int)k, rows, kp);
    } else {
        launch_transpose_i8(b, ldb, (int)k, (int)n, rows, kp, (int)kp, s);
    }
    NNOPS_LAUNCH(rowsum_i8, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, rows, kp, (int)n, (int)k, 0,
                       sums);
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}

extern "C" size_t nnops_hip_gemm_i8_workspace_size(const NnopsGemmI8Args* g)
{
    if (g == nullptr) {
        return 0;
    }
    return plan_workspace(*g).total;
}

extern "C" int nnops_hip_gemm_i8(const NnopsGemmI8Args* g, void* workspace, size_t ws_bytes, void* stream)
{
    const TimingDisarm disarm;
    if (g == nullptr || g->m < 0 || g->n < 0 || g->k < 0) {
        return NNOPS_INVALID_ARGUMENT;
    }
    if (g->m == 0 || g->n == 0) {
        return NNOPS_OK;
    }
    if (g->a == nullptr || g->b == nullptr || g->c == nullptr) {
        return NNOPS_INVALID_ARGUMENT;
    }
    const bool fp_out = g->out_kind == NNOPS_OUT_F32 || g->out_kind == NNOPS_OUT_F16;
    if (g->out_kind != NNOPS_OUT_S32 && g->out_kind != NNOPS_OUT_S8 && g->out_kind != NNOPS_OUT_U8 && !fp_out) {
        return NNOPS_UNSUPPORTED;
    }
    if (g->float_ep && g->out_kind == NNOPS_OUT_S32) {
        return NNOPS_UNSUPPORTED;
    }
    if (g->act < NNOPS_ACT_NONE || g->act > NNOPS_ACT_RELU6 ||
        (!fp_out && g->act != NNOPS_ACT_NONE && g->act != NNOPS_ACT_RELU && g->act != NNOPS_ACT_GELU)) {
        return NNOPS_UNSUPPORTED;
    }
    if ((fp_out && g->bias != nullptr) || (!fp_out && g->bias_fp != nullptr)) {
        return NNOPS_INVALID_ARGUMENT;   // an f32/f16 destination takes its bias in its own type
    }
    // int32 accumulate: |sum| <= K * 128 * 255 must stay below 2^31.
    if (g->k > 65535 || g->m > INT32_MAX || g->n > INT32_MAX) {
        return NNOPS_UNSUPPORTED;
    }
    const int64_t min_lda = g->trans_a ? g->m : g->k;
    const int64_t min_ldb = g->trans_b ? g->k : g->n;
    if (g->lda < min_lda || g->ldb < min_ldb || g->ldc < g->n) {
        return NNOPS_INVALID_ARGUMENT;
    }
    const WsPlan w = plan_workspace(*g);
    if (w.total > 0 && (workspace == nullptr || ws_bytes < w.total)) {
        return NNOPS_NOT_INITIALIZED;
    }
    if ((uintptr_t)workspace % 16 != 0) {
        return NNOPS_INVALID_ARGUMENT;   // staged operands and partials are 16-byte vectors
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* ws = static_cast<char*>(workspace);

    GemmI8Kern k{};
    k.m = (int)g->m;
    k.n = (int)g->n;
    k.k = (int)g->k;
    k.c = g->c;
    k.ldc_bytes = g->ldc * out_elem_bytes(g->out_kind);
    k.a_xor = g->a_u8 ? 0x80808080u : 0u;

    // k-contiguous operands (stage a transposed copy where needed)
    if (g->trans_a) {
        int8_t* at = reinterpret_cast<int8_t*>(ws + w.a_t);
        launch_transpose_i8(static_cast<const int8_t*>(g->a), g->lda, (int)g->k, (int)g->m, at, (int64_t)w.kp,
                            (int)w.kp, s);
        k.a = at;
        k.lda = w.kp;
    } else {
        k.a = static_cast<const int8_t*>(g->a);
        k.lda = g->lda;
    }
    if (w.kn.cpl != 0 || w.ring.trb) {
        k.b = g->b;               // [K,N], consumed in place by the column GEMV or the TRB ring
        k.ldb = g->ldb;
    } else if (!g->trans_b) {
        int8_t* bt = reinterpret_cast<int8_t*>(ws + w.b_t);
        launch_transpose_i8(g->b, g->ldb, (int)g->k, (int)g->n, bt, (int64_t)w.kp, (int)w.kp, s);
        k.b = bt;
        k.ldb = w.kp;
    } else {
        k.b = g->b;
        k.ldb = g->ldb;
    }

    // zero-point compensation terms
    EpiParams& e = k.ep;
    e.bias = g->bias;
    e.s_a = g->s_a; e.s_a_scalar = g->s_a_scalar;
    e.zp_a = g->zp_a; e.zp_a_scalar = g->zp_a_scalar;
    e.s_b = g->s_b; e.s_b_scalar = g->s_b_scalar;
    e.zp_b = g->zp_b; e.zp_b_scalar = g->zp_b_scalar;
    e.s_out_rows = g->s_out_rows; e.zp_out_rows = g->zp_out_rows;
    e.s_out = g->s_out; e.zp_out = g->zp_out;
    e.k = (int32_t)g->k;
    e.out_kind = g->out_kind;
    e.act = g->act;
    e.round_even = g->round_even;
    e.float_ep = g->float_ep;
    e.min_clip = g->min_clip;
    e.max_clip = g->max_clip;
    e.add_to = g->add_to;
    e.residual_pre = g->residual_pre;
    e.bias_fp = fp_out ? g->bias_fp : nullptr;
    e.act_alpha = g->act_alpha;
    e.act_beta = g->act_beta;
    if (fp_out) {
        e.float_ep = 0;
        e.round_even = 0;
    }
    e.a_off = g->a_u8 ? -128 : 0;
    const bool need_rb = g->a_u8 || g->zp_a != nullptr || g->zp_a_scalar != 0;
    const bool need_ra = g->zp_b != nullptr || g->zp_b_scalar != 0;
    e.compensate = need_ra || need_rb;
    if (need_rb && g->b_col_sums != nullptr) {
        e.r_b = g->b_col_sums;
    } else if (need_rb) {
        int32_t* rb = reinterpret_cast<int32_t*>(ws + w.r_b);
        NNOPS_LAUNCH(rowsum_i8, dim3((unsigned)((g->n + 3) / 4)), dim3(256), 0, s, k.b, k.ldb,
                           (int)g->n, (int)g->k, 0, rb);
        e.r_b = rb;
    }
    if (need_ra) {
        int32_t* ra = reinterpret_cast<int32_t*>(ws + w.r_a);
        NNOPS_LAUNCH(rowsum_i8, dim3((unsigned)((g->m + 3) / 4)), dim3(256), 0, s, k.a, k.lda,
                           (int)g->m, (int)g->k, (int)g->a_u8, ra);
        e.r_a = ra;
    }

    const bool aligned = aligned16(k.a, k.lda) && aligned16(k.b, k.ldb) && (g->k % 16 == 0);
    const bool fullk = aligned && (g->k % 64 == 0);
    const int epi = choose_epi(*g, e);
    if (w.kn.cpl != 0) {
        launch_kn(k, w.kn, reinterpret_cast<int32_t*>(ws + w.part), reinterpret_cast<uint64_t*>(ws + w.flag), s);
    } else if (g->m <= 16 && aligned && g->k % 64 == 0 && gemv_lds_ok(*g)) {
        NNOPS_LAUNCH((gemv_i8_lds<4>), dim3((unsigned)((g->n + 15) / 16)), dim3(256), 0, s, k);
    } else if (g->m <= 4 && aligned) {
        const bool flip = k.a_xor != 0u;
        // two rows per wave from M = 3: halves the A re-reads per weight byte
        const int rsel = g->m >= 3 ? 2 : 1;
#define NNOPS_ROWS_R(MT, R)                                                                         \
        {                                                                                           \
            const unsigned blocks = (unsigned)((g->n + 4 * R - 1) / (4 * R));                      \
            if (flip) {                                                                             \
                NNOPS_LAUNCH((gemv_i8_rows<MT, R, true>), dim3(blocks), dim3(256), 0, s, k);  \
            } else {                                                                                \
                NNOPS_LAUNCH((gemv_i8_rows<MT, R, false>), dim3(blocks), dim3(256), 0, s, k); \
            }                                                                                       \
        }
#define NNOPS_ROWS(MT)                                                                              \
        if (rsel == 2) NNOPS_ROWS_R(MT, 2) else NNOPS_ROWS_R(MT, 1)
        if (g->m == 1) {
            NNOPS_ROWS(1)
        } else if (g->m == 2) {
            NNOPS_ROWS(2)
        } else {
            NNOPS_ROWS(4)
        }
#undef NNOPS_ROWS_R
#undef NNOPS_ROWS
    } else if (g->m <= 16) {
        const unsigned blocks = (unsigned)((g->n + 15) / 16);
        if (aligned) {
            NNOPS_LAUNCH((gemv_i8_mfma<4, true>), dim3(blocks), dim3(256), 0, s, k);
        } else {
            NNOPS_LAUNCH((gemv_i8_mfma<4, false>), dim3(blocks), dim3(256), 0, s, k);
        }
    } else if (w.ring.mode >= 0) {
        launch_ring(k, w.ring, reinterpret_cast<int32_t*>(ws + w.part), s);
    } else if (g->m >= 1024 && g->n >= 1024) {
        launch_gemm<256, 256, 2, 2, 1>(k, aligned, fullk, epi, s);
    } else if (g->m >= 64) {
        launch_gemm<128, 128, 2, 2, 2>(k, aligned, fullk, epi, s);
    } else {
        launch_gemm<32, 64, 1, 2, 4>(k, aligned, fullk, epi, s);
    }
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}

// ---------------------------------------------------------------------------
// The ring over f16 operands (nnops_hip_gemm_fp's large shapes): the same
// byte staging, K and the row pitches in bytes; B [N][K] rows in place, or a
// [K][N] B transposed into the workspace first. RING_FP writes alpha * acc
// straight to C; K splits write f32 partials that ring_f16_reduce sums.
// ---------------------------------------------------------------------------
namespace nnops_amd {
namespace {

struct F16Plan {
    RingPlan ring;          // mode < 0: the ring does not take the call
    bool stage_b = false;
    int64_t kp = 0;         // staged B row bytes
    size_t part_off = 0, total = 0;
};

F16Plan plan_f16(const NnopsGemmFpArgs& g)
{
    F16Plan f;
    if (!g.in_f16 || g.m < 64 || 2 * g.k > INT32_MAX || g.m > INT32_MAX || g.n > INT32_MAX) {
        return f;
    }
    NnopsGemmI8Args x{};
    x.m = g.m;
    x.n = g.n;
    x.k = 2 * g.k;
    x.trans_b = 1;
    x.a = g.a;
    x.lda = 2 * g.lda;
    x.c = g.c;
    x.ldc = g.ldc;
    x.out_kind = g.out_f16 ? NNOPS_OUT_F16 : NNOPS_OUT_F32;
    x.act = NNOPS_ACT_NONE;
    x.s_a_scalar = g.alpha;
    x.s_b_scalar = 1.0f;
    const int8_t* b = static_cast<const int8_t*>(g.b);
    int64_t ldb = 2 * g.ldb;
    size_t off = 0;
    if (!g.trans_b) {
        f.stage_b = true;
        f.kp = (2 * g.k + 127) / 128 * 128;
        off += align_up((size_t)g.n * (size_t)f.kp);
        b = nullptr;          // the staged copy: 256-byte aligned, 128-byte rows
        ldb = f.kp;
    }
    f.ring = plan_ring(x, static_cast<const int8_t*>(g.a), x.lda, b, ldb);
    if (f.ring.mode != RING_FP && f.ring.mode != RING_PART) {
        f.ring = RingPlan{};
        return f;
    }
    // f32 partials cost 8 bytes of traffic per output and split: where
    // 128 x 256 tiles alone nearly fill the CUs, take them unsplit (512 x
    // 14336 x 4096: 89.6 us split in two over 256 x 256 tiles)
    const int64_t tiles128 = ((g.m + 127) / 128) * ((g.n + 255) / 256);
    const bool c_ok = (uintptr_t)g.c % 16 == 0 && (g.ldc * (g.out_f16 ? 2 : 4)) % 16 == 0;
    if (f.ring.splits > 1 && g.m > 128 && tiles128 >= 192 && c_ok) {
        f.ring.bm = 128;
        f.ring.bn = 256;
        f.ring.splits = 1;
        f.ring.mode = RING_FP;
    }
    if (f.ring.mode == RING_PART) {
        f.part_off = off;
        off += align_up((size_t)f.ring.splits * (size_t)g.m * (size_t)g.n * 4);
    }
    f.total = off;
    return f;
}

}  // namespace

bool ring_gemm_f16_ok(const NnopsGemmFpArgs& g)
{
    return plan_f16(g).ring.mode >= 0;
}

size_t ring_gemm_f16_workspace(const NnopsGemmFpArgs& g)
{
    // the destination's alignment (which a size query may not see) picks
    // between the fused output and the split partials: room for either
    NnopsGemmFpArgs x = g;
    const size_t a = plan_f16(x).total;
    x.c = reinterpret_cast<void*>(uintptr_t{2});
    return std::max(a, plan_f16(x).total);
}

int ring_gemm_f16(const NnopsGemmFpArgs& g, void* workspace, size_t ws_bytes, hipStream_t s)
{
    const F16Plan f = plan_f16(g);
    if (f.ring.mode < 0) {
        return NNOPS_UNSUPPORTED;
    }
    if (f.total > 0 && (workspace == nullptr || ws_bytes < f.total)) {
        return NNOPS_NOT_INITIALIZED;
    }
    if ((uintptr_t)workspace % 16 != 0) {
        return NNOPS_INVALID_ARGUMENT;   // staged operands and partials are 16-byte vectors
    }
    char* ws = static_cast<char*>(workspace);
    GemmI8Kern k{};
    k.m = (int)g.m;
    k.n = (int)g.n;
    k.k = (int)(2 * g.k);
    k.a = static_cast<const int8_t*>(g.a);
    k.lda = 2 * g.lda;
    k.c = g.c;
    k.ldc_bytes = g.ldc * (g.out_f16 ? 2 : 4);
    if (f.stage_b) {
        uint16_t* bt = reinterpret_cast<uint16_t*>(ws);
        const dim3 grid((unsigned)((g.n + 63) / 64), (unsigned)((f.kp / 2 + 63) / 64));
        NNOPS_LAUNCH(transpose_b16, grid, dim3(256), 0, s, static_cast<const uint16_t*>(g.b), g.ldb,
                           (int)g.k, (int)g.n, bt, f.kp / 2, (int)(f.kp / 2));
        k.b = reinterpret_cast<const int8_t*>(bt);
        k.ldb = f.kp;
    } else {
        k.b = static_cast<const int8_t*>(g.b);
        k.ldb = 2 * g.ldb;
    }
    EpiParams& e = k.ep;
    e.s_a_scalar = g.alpha;
    e.s_b_scalar = 1.0f;
    e.out_kind = g.out_f16 ? NNOPS_OUT_F16 : NNOPS_OUT_F32;
    e.act = NNOPS_ACT_NONE;
    e.min_clip = -INFINITY;
    e.max_clip = INFINITY;
    launch_ring<true>(k, f.ring, reinterpret_cast<int32_t*>(ws + f.part_off), s);
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}

}  // namespace nnops_amd
