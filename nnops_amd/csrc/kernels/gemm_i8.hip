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
//   gemv_i8_mfma   M <= 16: one 16-column slice of B per block, K split over
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

template <int BM, int BN, int WM, int WN, bool ALIGNED>
__global__ __launch_bounds__(WM * WN * 64, 1) void gemm_i8_mfma(GemmI8Kern p)
{
    constexpr int T = WM * WN * 64;
    constexpr int TM = BM / WM;           // wave tile rows
    constexpr int TN = BN / WN;           // wave tile cols
    constexpr int FM = TM / 32;           // 32x32 fragments per wave
    constexpr int FN = TN / 32;
    constexpr int CA = BM * (kBK / 16) / T;   // 16-byte chunks per thread per stage
    constexpr int CB = BN * (kBK / 16) / T;
    static_assert(CA >= 1 && CB >= 1 && CA * T == BM * 4 && CB * T == BN * 4, "tile/threads");

    __shared__ __attribute__((aligned(16))) int8_t lds_a[2][BM * kLdsRow];
    __shared__ __attribute__((aligned(16))) int8_t lds_b[2][BN * kLdsRow];

    int tm, tn;
    tile_coords((p.m + BM - 1) / BM, (p.n + BN - 1) / BN, tm, tn);
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm0 = (wave / WN) * TM;
    const int wn0 = (wave % WN) * TN;

    // Per-thread global source rows for the stage loads (clamped into range:
    // rows past M/N are computed but never stored).
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
    auto load_stage = [&](int k0) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            ra[i] = load16_a<ALIGNED>(a_src[i], k0 + a_kc[i], p.k, p.a_xor);
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            rb[i] = load16<ALIGNED>(b_src[i], k0 + b_kc[i], p.k);
        }
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            *reinterpret_cast<v4i*>(&lds_a[buf][a_lds[i]]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            *reinterpret_cast<v4i*>(&lds_b[buf][b_lds[i]]) = rb[i];
        }
    };

    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            acc[i][j] = v16i{0};
        }
    }

    const int kt = (p.k + kBK - 1) / kBK;
    load_stage(0);
    store_stage(0);
    __syncthreads();

    const int frag_row = lane & 31;
    const int frag_k = (lane >> 5) * 16;
    for (int t = 0; t < kt; ++t) {
        const int cur = t & 1;
        if (t + 1 < kt) {
            load_stage((t + 1) * kBK);
        }
#pragma unroll
        for (int ks = 0; ks < kBK; ks += 32) {
            v4i fa[FM], fb[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                fa[i] = *reinterpret_cast<const v4i*>(
                    &lds_a[cur][(wm0 + i * 32 + frag_row) * kLdsRow + ks + frag_k]);
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                fb[j] = *reinterpret_cast<const v4i*>(
                    &lds_b[cur][(wn0 + j * 32 + frag_row) * kLdsRow + ks + frag_k]);
            }
#pragma unroll
            for (int i = 0; i < FM; ++i) {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (t + 1 < kt) {
            store_stage(cur ^ 1);
        }
        __syncthreads();
    }

    // Output pass. 32x32 accumulator layout: lane holds column (lane & 31) and
    // rows 8*(r/4) + 4*(lane/32) + (r%4) for r in 0..15.
    const int ebytes = out_elem_bytes(p.ep.out_kind);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn0 + j * 32 + (lane & 31);
        if (n >= p.n) {
            continue;
        }
        const EpiCol col = epi_col(p.ep, n);
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < p.m) {
                    const EpiRow row = epi_row(p.ep, m);
                    char* crow = static_cast<char*>(p.c) + (int64_t)m * p.ldc_bytes;
                    (void)ebytes;
                    epi_store(p.ep, row, col, acc[i][j][r], crow, n);
                }
            }
        }
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
// Prepasses
// ---------------------------------------------------------------------------
// dst[c][r] = src[r][c] for r < R, c < C; dst columns r in [R, Rp) are zeroed.
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

// ---------------------------------------------------------------------------
// Host side: workspace plan and dispatch.
// ---------------------------------------------------------------------------
constexpr size_t kAlign = 256;
inline size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }
inline int64_t round16(int64_t x) { return (x + 15) / 16 * 16; }

struct WsPlan {
    size_t r_a = 0, r_b = 0, a_t = 0, b_t = 0, total = 0;
    int64_t kp = 0;
};

WsPlan plan_workspace(const NnopsGemmI8Args& g)
{
    WsPlan w;
    size_t off = 0;
    w.kp = round16(g.k);
    w.r_a = off; off += align_up((size_t)g.m * 4);
    w.r_b = off; off += align_up((size_t)g.n * 4);
    if (g.trans_a) {
        w.a_t = off; off += align_up((size_t)g.m * (size_t)w.kp);
    }
    if (!g.trans_b) {
        w.b_t = off; off += align_up((size_t)g.n * (size_t)w.kp);
    }
    w.total = off;
    return w;
}

inline bool aligned16(const void* p, int64_t ld) { return ((uintptr_t)p % 16 == 0) && (ld % 16 == 0); }

template <int BM, int BN, int WM, int WN>
void launch_gemm(const GemmI8Kern& k, bool aligned, hipStream_t s)
{
    const int tiles = ((k.m + BM - 1) / BM) * ((k.n + BN - 1) / BN);
    if (aligned) {
        hipLaunchKernelGGL((gemm_i8_mfma<BM, BN, WM, WN, true>), dim3(tiles), dim3(WM * WN * 64), 0, s, k);
    } else {
        hipLaunchKernelGGL((gemm_i8_mfma<BM, BN, WM, WN, false>), dim3(tiles), dim3(WM * WN * 64), 0, s, k);
    }
}

}  // namespace
}  // namespace nnops_amd

using namespace nnops_amd;

extern "C" size_t nnops_hip_gemm_i8_workspace_size(const NnopsGemmI8Args* g)
{
    if (g == nullptr) {
        return 0;
    }
    return plan_workspace(*g).total;
}

extern "C" int nnops_hip_gemm_i8(const NnopsGemmI8Args* g, void* workspace, size_t ws_bytes, void* stream)
{
    if (g == nullptr || g->m < 0 || g->n < 0 || g->k < 0) {
        return NNOPS_INVALID_ARGUMENT;
    }
    if (g->m == 0 || g->n == 0) {
        return NNOPS_OK;
    }
    if (g->a == nullptr || g->b == nullptr || g->c == nullptr) {
        return NNOPS_INVALID_ARGUMENT;
    }
    if (g->out_kind != NNOPS_OUT_S32 && g->out_kind != NNOPS_OUT_S8 && g->out_kind != NNOPS_OUT_U8) {
        return NNOPS_UNSUPPORTED;
    }
    if (g->float_ep && g->out_kind == NNOPS_OUT_S32) {
        return NNOPS_UNSUPPORTED;
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
        dim3 grid((unsigned)((g->m + 63) / 64), (unsigned)((w.kp + 63) / 64));
        hipLaunchKernelGGL(transpose_i8, grid, dim3(256), 0, s, static_cast<const int8_t*>(g->a), g->lda,
                           (int)g->k, (int)g->m, at, (int64_t)w.kp, (int)w.kp);
        k.a = at;
        k.lda = w.kp;
    } else {
        k.a = static_cast<const int8_t*>(g->a);
        k.lda = g->lda;
    }
    if (!g->trans_b) {
        int8_t* bt = reinterpret_cast<int8_t*>(ws + w.b_t);
        dim3 grid((unsigned)((g->n + 63) / 64), (unsigned)((w.kp + 63) / 64));
        hipLaunchKernelGGL(transpose_i8, grid, dim3(256), 0, s, g->b, g->ldb, (int)g->k, (int)g->n, bt,
                           (int64_t)w.kp, (int)w.kp);
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
    e.a_off = g->a_u8 ? -128 : 0;
    const bool need_rb = g->a_u8 || g->zp_a != nullptr || g->zp_a_scalar != 0;
    const bool need_ra = g->zp_b != nullptr || g->zp_b_scalar != 0;
    e.compensate = need_ra || need_rb;
    if (need_rb) {
        int32_t* rb = reinterpret_cast<int32_t*>(ws + w.r_b);
        hipLaunchKernelGGL(rowsum_i8, dim3((unsigned)((g->n + 3) / 4)), dim3(256), 0, s, k.b, k.ldb,
                           (int)g->n, (int)g->k, 0, rb);
        e.r_b = rb;
    }
    if (need_ra) {
        int32_t* ra = reinterpret_cast<int32_t*>(ws + w.r_a);
        hipLaunchKernelGGL(rowsum_i8, dim3((unsigned)((g->m + 3) / 4)), dim3(256), 0, s, k.a, k.lda,
                           (int)g->m, (int)g->k, (int)g->a_u8, ra);
        e.r_a = ra;
    }

    const bool aligned = aligned16(k.a, k.lda) && aligned16(k.b, k.ldb) && (g->k % 16 == 0);
    if (g->m <= 16) {
        const unsigned blocks = (unsigned)((g->n + 15) / 16);
        if (aligned) {
            hipLaunchKernelGGL((gemv_i8_mfma<4, true>), dim3(blocks), dim3(256), 0, s, k);
        } else {
            hipLaunchKernelGGL((gemv_i8_mfma<4, false>), dim3(blocks), dim3(256), 0, s, k);
        }
    } else if (g->m >= 1024 && g->n >= 1024) {
        launch_gemm<256, 256, 2, 2>(k, aligned, s);
    } else if (g->m >= 64) {
        launch_gemm<128, 128, 2, 2>(k, aligned, s);
    } else {
        launch_gemm<32, 64, 1, 2>(k, aligned, s);
    }
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}
