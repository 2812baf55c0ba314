// Q4_1-weight GEMM / GEMV on gfx950 (llama.cpp block_q4_1: f16 d, f16 m, 16
// nibble bytes; value j = d * q_j + m, q_j the low nibble of byte j for j < 16
// and the high nibble of byte j-16 otherwise).
//
// Kernels
//   gemv_q4_1_pipe  blocks along K ([N][K/32], Linear/GGUF form), K = 4096,
//                   M <= 2 per launch: each wave DMAs its 4 rows (one
//                   contiguous 10 KiB span) into LDS and decodes each (row,
//                   block half) as its pieces land; nibbles widened with the
//                   0x54 exponent trick (f16 0x54qq = 64 + q/16) and dotted
//                   with v_dot2_f32_f16 against A. Bound: HBM.
//   gemv_q4_1_lds,  the same decode for the other [N][K/32] GEMV shapes (rows
//   gemv_q4_1_rows, staged in LDS, or read straight from HBM; f32 A).
//   gemv_q4_1_nk
//   gemv_q4_1_kn_dma  blocks along N ([K][N/32]), raw rows, f16 A, M <= 2 per
//                   launch: 640-byte row segments (32 blocks) of a K range DMAed
//                   into an LDS ring, nibbles widened by v_perm / and-or into
//                   f16 pairs of two rows and dotted with (a d) pairs; the K
//                   splits of a column group summed by its last-arriving
//                   workgroup in the same launch. Bound: HBM.
//   gemv_q4_1_bcm   the prepacked planes of blocks along N, f16 A, M <= 2 per
//                   launch: a workgroup per block column (32 columns) over the
//                   whole of K, streaming its two contiguous runs as 1 KiB
//                   wave loads; one launch, no workspace. Bound: HBM.
//   gemv_q4_1_kn    blocks along N with f32 A or odd K (raw rows or the
//                   prepacked planes): a lane owns one nibble dword (8
//                   columns) of a block, 16 rows of loads in flight; waves and
//                   workgroups split K, partial planes summed by reduce_q4_1.
//   gemm_q4_1_ring  larger M, f16 A, blocks along K, K % 64 == 0: a 4-stage
//                   LDS ring filled by DMA (A and the raw Q4_1 bytes), 8 waves
//                   of 128 x 32, B decoded per lane into MFMA operands with
//                   packed f16 math, v_mfma_f32_32x32x16_f16. Bound: MFMA.
//   gemm_q4_1_kn_ring  the same ring for blocks along N (raw rows or the
//                   prepacked planes), each lane decoding its column at 8
//                   consecutive k rows.
//   gemm_q4_1_mfma  the other GEMM shapes: B tiles decoded to f16 (d*q + m in
//                   f32, rounded once) into LDS, A tiles staged k-contiguous.
//   prepack_q4_1_kn prepackWeights of a blocks-along-N weight: its nibble
//                   plane and its d|m plane.
#include "fp_out.hpp"


#include <atomic>
#include <utility>

namespace nnops_amd {
namespace {

typedef int v4i_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef unsigned int v2u32 __attribute__((ext_vector_type(2)));

struct Q41Kern {
    const void* a;       // f16 or f32 [M][lda]
    const uint8_t* b;
    void* c;
    float* partial;      // [splits][M][N] (kn form)
    int m, n, k;
    int64_t lda, ldc, ldb;   // lda/ldc in elements, ldb in bytes
    int out_f16;
    int splits;
    const uint32_t* bdm; // SoA d|m plane, block column j at j * ldbdm (prepacked blocks along N)
    int64_t ldbdm;       // u32 elements
    FpOut fo;            // the fused gated combine (gemm_q4_1_ring with GATED)
    const float* row_scale;  // SPLIT ring: [M] power-of-two factor of each row of A
    int64_t plane;           // SPLIT ring: bytes from the hi plane of A to the lo plane
};

__device__ __forceinline__ float h2f(uint32_t bits16)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// The prepacked blocks-along-N planes (nnops_hip_prepack_q4_1), one block
// column (32 columns) after another: block column j of the nibble plane is
// p.ldb = ceil(K/8) * 128 bytes, its group of 8 rows r / 8 the 128 bytes at
// (r / 8) * 128, holding nibble dword d of row r at 32 d + 4 (r % 8); block
// column j of the d|m plane is p.ldbdm dwords, row r's (f16 d, f16 m) at r.
__device__ __forceinline__ const uint8_t* soa_group(const Q41Kern& p, int64_t j, int64_t r)
{
    return p.b + j * p.ldb + (r >> 3) * 128;
}
__device__ __forceinline__ uint32_t soa_dm(const Q41Kern& p, int64_t j, int64_t r)
{
    return p.bdm[j * p.ldbdm + r];
}

template <bool AF16>
__device__ __forceinline__ float load_a(const Q41Kern& p, int m, int k)
{
    if constexpr (AF16) {
        return (float)static_cast<const _Float16*>(p.a)[(int64_t)m * p.lda + k];
    } else {
        return static_cast<const float*>(p.a)[(int64_t)m * p.lda + k];
    }
}

__device__ __forceinline__ void store_out(const Q41Kern& p, int m, int n, float v)
{
    if (p.out_f16) {
        __builtin_nontemporal_store((_Float16)v, static_cast<_Float16*>(p.c) + (int64_t)m * p.ldc + n);
    } else {
        __builtin_nontemporal_store(v, static_cast<float*>(p.c) + (int64_t)m * p.ldc + n);
    }
}

// Workgroup barrier without a memory fence: the ring's DMA stays in flight
// (its landing is awaited with explicit vmcnt waits); only LDS accesses are
// kept from moving across it.
__device__ __forceinline__ void q_block_barrier()
{
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// (x & m) | o in one v_and_or_b32 (the compiler splits the pair otherwise)
__device__ __forceinline__ uint32_t and_or_u32(uint32_t x, uint32_t m, uint32_t o)
{
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(m), "v"(o));
    return r;
}

// Buffer resource over [base, base + bytes): loads past the end read 0.
#define NNOPS_LPTR(x) ((__attribute__((address_space(3))) void*)(x))
#if __HIP_DEVICE_COMPILE__
typedef __amdgpu_buffer_rsrc_t QBufRsrc;
#else
struct QBufRsrc {
    int w[4];
};
#endif

__device__ __forceinline__ QBufRsrc q_buffer_rsrc(const void* base, uint32_t bytes)
{
#if __HIP_DEVICE_COMPILE__
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
#else
    (void)base, (void)bytes;
    return QBufRsrc{};
#endif
}

// 16-byte store / load with the sc1 cache policy: coherent at device scope,
// the lowering of an agent-scope atomic store / load, without a cache-wide
// fence.
__device__ __forceinline__ void q_buffer_store16_sc1(QBufRsrc r, v4i v, int voff)
{
#if __HIP_DEVICE_COMPILE__
    __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, 0, 16);
#else
    (void)r, (void)v, (void)voff;
#endif
}

__device__ __forceinline__ void q_buffer_store8_sc1(QBufRsrc r, uint64_t v, int voff)
{
#if __HIP_DEVICE_COMPILE__
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32, v), r, voff, 0, 16);
#else
    (void)r, (void)v, (void)voff;
#endif
}

__device__ __forceinline__ uint64_t q_buffer_load8_sc1(QBufRsrc r, int voff)
{
#if __HIP_DEVICE_COMPILE__
    return __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 16));
#else
    (void)r, (void)voff;
    return 0;
#endif
}

__device__ __forceinline__ v4i q_buffer_load16_sc1(QBufRsrc r, int voff)
{
#if __HIP_DEVICE_COMPILE__
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 16);
#else
    (void)r, (void)voff;
    return v4i{0, 0, 0, 0};
#endif
}

// AUX: the cache policy bits (2: non-temporal, for weights read once)
template <int AUX = 0>
__device__ __forceinline__ void q_buffer_load_lds16(QBufRsrc r, uint8_t* lds, int voff, int soff)
{
#if __HIP_DEVICE_COMPILE__
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, NNOPS_LPTR(lds), 16, voff, soff, 0, AUX);
#else
    (void)r, (void)lds, (void)voff, (void)soff;
#endif
}

// ---------------------------------------------------------------------------
// GEMV, blocks along K.
// ---------------------------------------------------------------------------
constexpr int kNkRowsPerWave = 4;
constexpr int kNkWaves = 4;
constexpr int kNkChunkBlocks = 256;   // K chunk staged in LDS: 256 blocks = 8192 values

template <int MT, bool AF16>
__global__ __launch_bounds__(256) void gemv_q4_1_nk(Q41Kern p)
{
    // A chunk, as f16 pairs (AF16) or f32, plus per-block sums sum_j a_j.
    __shared__ uint32_t lds_a[MT][AF16 ? kNkChunkBlocks * 16 : kNkChunkBlocks * 32];
    __shared__ float lds_asum[MT][kNkChunkBlocks];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kNkWaves + wave) * kNkRowsPerWave;
    const int nb = (p.k + 31) / 32;

    float acc[kNkRowsPerWave][MT];
#pragma unroll
    for (int r = 0; r < kNkRowsPerWave; ++r) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            acc[r][m] = 0.0f;
        }
    }

    for (int cb0 = 0; cb0 < nb; cb0 += kNkChunkBlocks) {
        const int cbn = min(kNkChunkBlocks, nb - cb0);
        __syncthreads();
        // Stage A[:, cb0*32 : (cb0+cbn)*32) (zero past K) and block sums.
        for (int i = threadIdx.x; i < MT * cbn; i += 256) {
            const int m = i / cbn;
            const int blk = i - m * cbn;
            const int kb = (cb0 + blk) * 32;
            float s = 0.0f;
            if constexpr (AF16) {
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int k = kb + 2 * j;
                    const _Float16 x0 = (m < p.m && k < p.k) ? static_cast<const _Float16*>(p.a)[(int64_t)m * p.lda + k] : (_Float16)0;
                    const _Float16 x1 = (m < p.m && k + 1 < p.k) ? static_cast<const _Float16*>(p.a)[(int64_t)m * p.lda + k + 1] : (_Float16)0;
                    s += (float)x0 + (float)x1;
                    lds_a[m][blk * 16 + j] = (uint32_t)__builtin_bit_cast(uint16_t, x0) |
                                             ((uint32_t)__builtin_bit_cast(uint16_t, x1) << 16);
                }
            } else {
#pragma unroll 8
                for (int j = 0; j < 32; ++j) {
                    const int k = kb + j;
                    const float x = (m < p.m && k < p.k) ? static_cast<const float*>(p.a)[(int64_t)m * p.lda + k] : 0.0f;
                    s += x;
                    lds_a[m][blk * 32 + j] = __float_as_uint(x);
                }
            }
            lds_asum[m][blk] = s;
        }
        __syncthreads();

        for (int blk = lane; blk < cbn; blk += 64) {
            uint32_t raw[kNkRowsPerWave][5];
#pragma unroll
            for (int r = 0; r < kNkRowsPerWave; ++r) {
                const int n = min(row0 + r, p.n - 1);
                const uint8_t* src = p.b + (int64_t)n * p.ldb + (int64_t)(cb0 + blk) * 20;
                const v4i_a4 x = __builtin_nontemporal_load(reinterpret_cast<const v4i_a4*>(src));
                raw[r][0] = (uint32_t)x.x;
                raw[r][1] = (uint32_t)x.y;
                raw[r][2] = (uint32_t)x.z;
                raw[r][3] = (uint32_t)x.w;
                raw[r][4] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(src + 16));
            }
#pragma unroll
            for (int r = 0; r < kNkRowsPerWave; ++r) {
                const float d = h2f(raw[r][0] & 0xffffu);
                const float mn = h2f(raw[r][0] >> 16);
                if constexpr (AF16) {
                    // h[p] = f16 pair (64 + q_2p/16, 64 + q_2p+1/16)
                    uint32_t h[16];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t q = raw[r][1 + i];
                        const uint32_t lo = q & 0x0f0f0f0fu;
                        const uint32_t hi = (q >> 4) & 0x0f0f0f0fu;
                        h[2 * i] = (lo & 0xffu) | ((lo << 8) & 0x00ff0000u) | 0x54005400u;
                        h[2 * i + 1] = ((lo >> 16) & 0xffu) | ((lo >> 8) & 0x00ff0000u) | 0x54005400u;
                        h[8 + 2 * i] = (hi & 0xffu) | ((hi << 8) & 0x00ff0000u) | 0x54005400u;
                        h[8 + 2 * i + 1] = ((hi >> 16) & 0xffu) | ((hi >> 8) & 0x00ff0000u) | 0x54005400u;
                    }
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        float s = 0.0f;
                        const uint32_t* ap = &lds_a[m][blk * 16];
#pragma unroll
                        for (int j = 0; j < 16; ++j) {
                            s = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, ap[j]),
                                                       __builtin_bit_cast(v2h, h[j]), s, false);
                        }
                        const float asum = lds_asum[m][blk];
                        // sum_j a_j (d q_j + mn) = 16 d (s - 64 asum) + mn asum
                        const float qsum = 16.0f * (s - 64.0f * asum);
                        acc[r][m] = fmaf(d, qsum, fmaf(mn, asum, acc[r][m]));
                    }
                } else {
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        float s = 0.0f;
                        const float* ap = reinterpret_cast<const float*>(&lds_a[m][blk * 32]);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const uint32_t q = raw[r][1 + i];
#pragma unroll
                            for (int b = 0; b < 4; ++b) {
                                s = fmaf(ap[4 * i + b], (float)((q >> (8 * b)) & 15u), s);
                                s = fmaf(ap[16 + 4 * i + b], (float)((q >> (8 * b + 4)) & 15u), s);
                            }
                        }
                        acc[r][m] = fmaf(d, s, fmaf(mn, lds_asum[m][blk], acc[r][m]));
                    }
                }
            }
        }
    }

    // Wave reduction of every (row, m) partial.
#pragma unroll
    for (int r = 0; r < kNkRowsPerWave; ++r) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float v = acc[r][m];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                v += __shfl_xor(v, off, 64);
            }
            acc[r][m] = v;
        }
    }
    if (lane < kNkRowsPerWave * MT) {
        const int r = lane / MT;
        const int m = lane - r * MT;
        float v = 0.0f;
#pragma unroll
        for (int rr = 0; rr < kNkRowsPerWave; ++rr) {
#pragma unroll
            for (int mm = 0; mm < MT; ++mm) {
                if (rr == r && mm == m) {
                    v = acc[rr][mm];
                }
            }
        }
        const int n = row0 + r;
        if (n < p.n && m < p.m) {
            store_out(p, m, n, v);
        }
    }
}

// ---------------------------------------------------------------------------
// GEMV v2, blocks along K, f16 A, M <= 2: no LDS. A wave owns R rows; lane l
// owns blocks l, l+64, ... of every row, reads those blocks' A values straight
// from global memory (L1/L2-resident: A is K*2 bytes), widens them to f16
// pairs and forms the block sums once, then streams its R rows' blocks
// (non-temporal dwordx4 + dword per block) and dots them on v_dot2_f32_f16.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t nib_pair(uint32_t nibs, uint32_t sel)
{
    // two nibble bytes -> f16 pair (0x54qq = 64 + q/16) via v_perm_b32
    return __builtin_amdgcn_perm(0x54545454u, nibs, sel);
}

template <int MT, int R>
__global__ __launch_bounds__(256) void gemv_q4_1_rows(Q41Kern p)
{
    constexpr int NB = 2;                    // blocks per lane per pass, all loads issued up front
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * 4 + wave) * R;
    if (n0 >= p.n) {
        return;
    }
    const int nb = (p.k + 31) / 32;
    const _Float16* A = static_cast<const _Float16*>(p.a);
    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            acc[r][m] = 0.0f;
        }
    }
    const bool a_vec = ((p.lda & 7) == 0) && (((uintptr_t)A & 15) == 0);
    const uint8_t* rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        rows[r] = p.b + (int64_t)min(n0 + r, p.n - 1) * p.ldb;
    }
    for (int b0 = 0; b0 < nb; b0 += 64 * NB) {
        uint32_t raw[NB][R][5];
        uint32_t ah[NB][MT][16];
        // weights first (the HBM stream), then this lane's A values (L1/L2)
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int blk = b0 + lane + 64 * u;
            const bool live = blk < nb;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint8_t* src = rows[r] + (int64_t)(live ? blk : 0) * 20;
                const v4i_a4 x = __builtin_nontemporal_load(reinterpret_cast<const v4i_a4*>(src));
                raw[u][r][0] = live ? (uint32_t)x.x : 0u;   // d = m = 0: a dead block adds 0
                raw[u][r][1] = (uint32_t)x.y;
                raw[u][r][2] = (uint32_t)x.z;
                raw[u][r][3] = (uint32_t)x.w;
                raw[u][r][4] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(src + 16));
            }
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int blk = b0 + lane + 64 * u;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const int mm = min(m, p.m - 1);
                const _Float16* arow = A + (int64_t)mm * p.lda + (int64_t)blk * 32;
                if (a_vec && blk * 32 + 32 <= p.k) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const v4i x = *reinterpret_cast<const v4i*>(arow + 8 * q);
                        ah[u][m][4 * q + 0] = (uint32_t)x.x;
                        ah[u][m][4 * q + 1] = (uint32_t)x.y;
                        ah[u][m][4 * q + 2] = (uint32_t)x.z;
                        ah[u][m][4 * q + 3] = (uint32_t)x.w;
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const int k = blk * 32 + 2 * j;
                        const uint32_t lo = k < p.k ? __builtin_bit_cast(uint16_t, arow[2 * j]) : 0u;
                        const uint32_t hi = k + 1 < p.k ? __builtin_bit_cast(uint16_t, arow[2 * j + 1]) : 0u;
                        ah[u][m][j] = lo | (hi << 16);
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            float asum[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                float sa = 0.0f;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    sa = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, ah[u][m][j]),
                                                __builtin_bit_cast(v2h, 0x3c003c00u), sa, false);
                }
                asum[m] = sa;
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float d = h2f(raw[u][r][0] & 0xffffu);
                const float mn = h2f(raw[u][r][0] >> 16);
                uint32_t h[16];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t lo = raw[u][r][1 + i] & 0x0f0f0f0fu;
                    const uint32_t hi = (raw[u][r][1 + i] >> 4) & 0x0f0f0f0fu;
                    h[2 * i] = nib_pair(lo, 0x04010400u);
                    h[2 * i + 1] = nib_pair(lo, 0x04030402u);
                    h[8 + 2 * i] = nib_pair(hi, 0x04010400u);
                    h[8 + 2 * i + 1] = nib_pair(hi, 0x04030402u);
                }
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    float sq = 0.0f;
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        sq = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, ah[u][m][j]),
                                                    __builtin_bit_cast(v2h, h[j]), sq, false);
                    }
                    // sum_j a_j (d q_j + mn) = 16 d (sq - 64 asum) + mn asum
                    const float qsum = 16.0f * (sq - 64.0f * asum[m]);
                    acc[r][m] = fmaf(d, qsum, fmaf(mn, asum[m], acc[r][m]));
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float v = acc[r][m];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                v += __shfl_xor(v, off, 64);
            }
            acc[r][m] = v;
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                if (n0 + r < p.n && m < p.m) {
                    store_out(p, m, n0 + r, acc[r][m]);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// GEMV v3, blocks along K, f16 A, M <= 2, rows of up to 128 blocks (K <= 4096
// per pass): each wave pulls its R rows into a private LDS region with
// global_load_lds_dwordx4 (1 KiB contiguous per instruction, so the HBM stream
// is perfectly coalesced), then every lane reads its own 20-byte blocks back
// from LDS. A wave only reads what it loaded itself: no block barrier.
// ---------------------------------------------------------------------------
#define NNOPS_GPTR(x) ((const __attribute__((address_space(1))) void*)(x))

template <int MT, int R>
__global__ __launch_bounds__(256) void gemv_q4_1_lds(Q41Kern p)
{
    constexpr int kRowBytes = 3072;                    // >= 128 blocks * 20 bytes, 3 DMA instructions
    __shared__ __attribute__((aligned(16))) uint8_t stage[4][R][kRowBytes];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * 4 + wave) * R;
    if (n0 >= p.n) {
        return;
    }
    const int nb = (p.k + 31) / 32;                     // host guarantees nb <= 128
    const int row_bytes = nb * 20;
    const _Float16* A = static_cast<const _Float16*>(p.a);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint8_t* row = p.b + (int64_t)min(n0 + r, p.n - 1) * p.ldb;
#pragma unroll
        for (int q = 0; q < kRowBytes / 1024; ++q) {
            const int off = q * 1024 + lane * 16;
            // chunks past the row re-read its start (kept in bounds, never used)
            const uint8_t* src = row + (off + 16 <= row_bytes ? off : 0);
            __builtin_amdgcn_global_load_lds(NNOPS_GPTR(src), NNOPS_LPTR(&stage[wave][r][q * 1024]), 16, 0, 2);
        }
    }
    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            acc[r][m] = 0.0f;
        }
    }
    // A for this lane's blocks while the weights land
    constexpr int NB = 2;
    uint32_t ah[NB][MT][16];
    const bool a_vec = ((p.lda & 7) == 0) && (((uintptr_t)A & 15) == 0);
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        const int blk = lane + 64 * u;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int mm = min(m, p.m - 1);
            const _Float16* arow = A + (int64_t)mm * p.lda + (int64_t)blk * 32;
            if (a_vec && blk * 32 + 32 <= p.k) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const v4i x = *reinterpret_cast<const v4i*>(arow + 8 * q);
                    ah[u][m][4 * q + 0] = (uint32_t)x.x;
                    ah[u][m][4 * q + 1] = (uint32_t)x.y;
                    ah[u][m][4 * q + 2] = (uint32_t)x.z;
                    ah[u][m][4 * q + 3] = (uint32_t)x.w;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int k = blk * 32 + 2 * j;
                    const uint32_t lo = k < p.k ? __builtin_bit_cast(uint16_t, arow[2 * j]) : 0u;
                    const uint32_t hi = k + 1 < p.k ? __builtin_bit_cast(uint16_t, arow[2 * j + 1]) : 0u;
                    ah[u][m][j] = lo | (hi << 16);
                }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0070 | (15 << 8));   // vmcnt(0): the wave's DMA landed
    asm volatile("" ::: "memory");
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        const int blk = lane + 64 * u;
        if (blk >= nb) {
            continue;
        }
        float asum[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float sa = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                sa = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, ah[u][m][j]),
                                            __builtin_bit_cast(v2h, 0x3c003c00u), sa, false);
            }
            asum[m] = sa;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t* bp = reinterpret_cast<const uint32_t*>(&stage[wave][r][blk * 20]);
            uint32_t raw[5];
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                raw[i] = bp[i];
            }
            const float d = h2f(raw[0] & 0xffffu);
            const float mn = h2f(raw[0] >> 16);
            uint32_t h[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo = raw[1 + i] & 0x0f0f0f0fu;
                const uint32_t hi = (raw[1 + i] >> 4) & 0x0f0f0f0fu;
                h[2 * i] = nib_pair(lo, 0x04010400u);
                h[2 * i + 1] = nib_pair(lo, 0x04030402u);
                h[8 + 2 * i] = nib_pair(hi, 0x04010400u);
                h[8 + 2 * i + 1] = nib_pair(hi, 0x04030402u);
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                float sq = 0.0f;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    sq = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, ah[u][m][j]),
                                                __builtin_bit_cast(v2h, h[j]), sq, false);
                }
                const float qsum = 16.0f * (sq - 64.0f * asum[m]);
                acc[r][m] = fmaf(d, qsum, fmaf(mn, asum[m], acc[r][m]));
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float v = acc[r][m];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                v += __shfl_xor(v, off, 64);
            }
            acc[r][m] = v;
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                if (n0 + r < p.n && m < p.m) {
                    store_out(p, m, n0 + r, acc[r][m]);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// GEMV, blocks along K, K = 4096 (128 blocks, 2560-byte rows), rows stored
// back to back: the pipelined form. A wave first loads its lanes' A (two
// blocks per lane, from L2), then DMAs its R rows as one contiguous span of
// 1 KiB pieces into LDS, and decodes each (row, block half) as soon as the
// pieces it needs have landed, so the decode ALU work overlaps the HBM stream
// instead of following it (every wave of the launch is resident at once).
// ---------------------------------------------------------------------------
//
// GATED: Linear's gated form with its output pass p.fo fused. p.n = 2 p.fo.n
// weight rows (gate rows, then value rows); a wave stages gate rows n0, n0 + 1
// and value rows p.fo.n + n0, p.fo.n + n0 + 1 (two 5 KiB spans) and combines
// its two outputs with fp_out_value, from the same f32 products the two-step
// form stages, so the bits are the two-step form's.
template <int MT, int R, bool GATED = false, bool OUT16 = false>
__global__ __launch_bounds__(256) void gemv_q4_1_pipe(Q41Kern p)
{
    constexpr int kRow = 128 * 20;
    constexpr int C = (R * kRow + 1023) / 1024;      // DMA pieces per wave
    static_assert(!GATED || R == 4, "gated: two gate and two value rows per wave");
    __shared__ __attribute__((aligned(16))) uint8_t stage[4][C * 1024];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nout = GATED ? p.fo.n : p.n;              // outputs (gated: half the weight rows)
    const int n0 = (blockIdx.x * 4 + wave) * (GATED ? R / 2 : R);
    if (n0 >= nout) {
        return;
    }
    // A first: its loads retire before the DMA pieces queued behind them
    const uint32_t* A = static_cast<const uint32_t*>(p.a);   // f16 pairs
    uint32_t ah[2][MT][16];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const v4i* src = reinterpret_cast<const v4i*>(A + (int64_t)min(m, p.m - 1) * (p.lda / 2) +
                                                          (lane + 64 * u) * 16);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const v4i x = src[q];
                ah[u][m][4 * q + 0] = (uint32_t)x.x;
                ah[u][m][4 * q + 1] = (uint32_t)x.y;
                ah[u][m][4 * q + 2] = (uint32_t)x.z;
                ah[u][m][4 * q + 3] = (uint32_t)x.w;
            }
        }
    }
    // every lane issues every piece (past the last row: a re-read of the
    // span's start), so the piece count, and the waits below, are static
    if constexpr (GATED) {
        // pieces 0-4: the gate rows' span, 5-9: the value rows' (2 x 2560 bytes each)
        const uint8_t* span[2] = {p.b + (int64_t)n0 * kRow, p.b + (int64_t)(nout + n0) * kRow};
        const int valid = min(R / 2, nout - n0) * kRow;
#pragma unroll
        for (int q = 0; q < C; ++q) {
            const int h = q < C / 2 ? 0 : 1;
            const int off = (q - h * (C / 2)) * 1024 + lane * 16;
            __builtin_amdgcn_global_load_lds(NNOPS_GPTR(span[h] + (off + 16 <= valid ? off : 0)),
                                             NNOPS_LPTR(&stage[wave][q * 1024]), 16, 0, 2);
        }
    } else {
        const uint8_t* first = p.b + (int64_t)n0 * kRow;
        const int valid = min(R, p.n - n0) * kRow;
#pragma unroll
        for (int q = 0; q < C; ++q) {
            const int off = q * 1024 + lane * 16;
            __builtin_amdgcn_global_load_lds(NNOPS_GPTR(first + (off + 16 <= valid ? off : 0)),
                                             NNOPS_LPTR(&stage[wave][q * 1024]), 16, 0, 2);
        }
    }
    // GATED: lane r * MT + m finishes output (m, n0 + r). Its two bias values
    // and the destination's current value (add_to) are loaded now, behind
    // the DMA pieces: three loads every lane issues, at clamped or stand-in
    // addresses where a value is absent, so the counts the waits below
    // allow for are fixed (XL), and widened only in the combine.
    constexpr int XL = GATED ? 3 : 0;
    using OutBits = std::conditional_t<OUT16, uint16_t, uint32_t>;
    OutBits x_bg{}, x_bu{}, x_old{};
    if constexpr (GATED) {
        // the waits count these loads as issued after the pieces: keep them there
        asm volatile("" ::: "memory");
        const FpOut& fo = p.fo;
        const int r = lane / MT, m = min(lane % MT, p.m - 1);
        const int n = min(n0 + min(r, R / 2 - 1), nout - 1);
        const OutBits* orow = reinterpret_cast<const OutBits*>(static_cast<const char*>(fo.out) +
                                                                (int64_t)m * fo.ld_out * sizeof(OutBits));
        const OutBits* bb = fo.bias != nullptr ? static_cast<const OutBits*>(fo.bias) : orow;
        const int nb = fo.bias != nullptr ? n : 0;
        x_bg = bb[nb];
        x_bu = bb[fo.bias != nullptr ? nout + n : 0];
        x_old = orow[n];
    }
    const v2h one = __builtin_bit_cast(v2h, 0x3c003c00u);
    float asum[2][MT];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float t = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                t = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, ah[u][m][j]), one, t, false);
            }
            asum[u][m] = t;
        }
    }
    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            acc[r][m] = 0.0f;
        }
    }
    auto phase = [&]<int RR, int U>() {
        // last byte this (row, half) needs, and the piece holding it
        constexpr int last = RR * kRow + (64 * U + 63) * 20 + 19;
        wait_vmcnt<C - 1 - last / 1024 + XL>();
        asm volatile("" ::: "memory");
        const uint32_t* bp = reinterpret_cast<const uint32_t*>(&stage[wave][RR * kRow + (lane + 64 * U) * 20]);
        uint32_t raw[5];
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            raw[i] = bp[i];
        }
        const float d = h2f(raw[0] & 0xffffu);
        const float mn = h2f(raw[0] >> 16);
        uint32_t h[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = raw[1 + i] & 0x0f0f0f0fu;
            const uint32_t hi = (raw[1 + i] >> 4) & 0x0f0f0f0fu;
            h[2 * i] = nib_pair(lo, 0x04010400u);
            h[2 * i + 1] = nib_pair(lo, 0x04030402u);
            h[8 + 2 * i] = nib_pair(hi, 0x04010400u);
            h[8 + 2 * i + 1] = nib_pair(hi, 0x04030402u);
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float sq = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                sq = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, ah[U][m][j]), __builtin_bit_cast(v2h, h[j]), sq,
                                            false);
            }
            const float qsum = 16.0f * (sq - 64.0f * asum[U][m]);
            acc[RR][m] = fmaf(d, qsum, fmaf(mn, asum[U][m], acc[RR][m]));
        }
    };
    [&]<int... I>(std::integer_sequence<int, I...>) {
        (phase.template operator()<I / 2, I % 2>(), ...);
    }(std::make_integer_sequence<int, 2 * R>{});
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float v = acc[r][m];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                v += __shfl_xor(v, off, 64);
            }
            acc[r][m] = v;
        }
    }
    if constexpr (GATED) {
        // lane r * MT + m finishes output (m, n0 + r) (gate product acc[r],
        // value acc[R/2 + r]; every lane holds the sums); lane m then writes
        // row m's pair as one 4-byte word where f16 allows: a 2-byte store
        // per output costs a read-modify-write each (1.2 us of the launch)
        static_assert(R / 2 == 2, "one f16 pair per row");
        const FpOut& fo = p.fo;
        const int r = lane / MT, m = lane % MT;
        // the early loads' bits as bias_at / fp_out_old read them (0 when absent)
        wait_vmcnt<0>();
        auto widen = [](OutBits v) {
            if constexpr (OUT16) {
                return (float)__builtin_bit_cast(_Float16, v);
            } else {
                return __builtin_bit_cast(float, v);
            }
        };
        const float pre_bg = fo.bias != nullptr ? widen(x_bg) : 0.0f;
        const float pre_bu = fo.bias != nullptr ? widen(x_bu) : 0.0f;
        const float pre_old = fp_out_reads_old(fo) ? widen(x_old) : 0.0f;
        float y = 0.0f;
#pragma unroll
        for (int rr = 0; rr < R / 2; ++rr) {
#pragma unroll
            for (int mm = 0; mm < MT; ++mm) {
                if (lane == rr * MT + mm) {
                    y = fp_out_value(fo, acc[rr][mm], acc[R / 2 + rr][mm], pre_old, pre_bg, pre_bu);
                }
            }
        }
        const float y1 = __shfl(y, lane + MT, 64);       // lane m: output (m, n0 + 1)
        if (r == 0 && m < p.m && n0 < nout) {
            char* orow = static_cast<char*>(fo.out) + (int64_t)m * fo.ld_out * (fo.out_f16 ? 2 : 4);
            _Float16* h = reinterpret_cast<_Float16*>(orow) + n0;
            if (n0 + 1 < nout && fo.out_f16 && ((uintptr_t)h & 3) == 0) {
                const _Float16 pr[2] = {(_Float16)y, (_Float16)y1};
                *reinterpret_cast<uint32_t*>(h) = __builtin_bit_cast(uint32_t, pr);
            } else {
                fp_out_store(fo, orow, n0, y);
                if (n0 + 1 < nout) {
                    fp_out_store(fo, orow, n0 + 1, y1);
                }
            }
        }
        return;
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                if (n0 + r < p.n && m < p.m) {
                    store_out(p, m, n0 + r, acc[r][m]);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// GEMV, blocks along N: partial[split][m][n].
// ---------------------------------------------------------------------------
template <int MT, bool AF16, bool SOA>
__global__ __launch_bounds__(256) void gemv_q4_1_kn(Q41Kern p)
{
    // Lane l owns nibble dword l & 3 of block (l >> 2) of the workgroup's 16
    // blocks: columns 4j .. 4j+3 (low nibbles) and 16+4j .. 16+4j+3 (high)
    // of the block. The 4 waves take interleaved k rows; per row a lane
    // loads the block's d|m dword and its nibble dword, 16 rows at a time.
    constexpr int U = 16;
    __shared__ float red[3][MT][8][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nblocks = (p.n + 31) / 32;
    const int bl = blockIdx.x * 16 + (lane >> 2);
    const int jq = lane & 3;
    const int split = blockIdx.y;
    // SOA splits start on a group of 8 rows
    const int kper = SOA ? ((p.k + p.splits - 1) / p.splits + 7) / 8 * 8 : (p.k + p.splits - 1) / p.splits;
    const int k0 = split * kper;
    const int k1 = min(p.k, k0 + kper);
    const bool live = bl < nblocks;
    const uint8_t* col = p.b + (int64_t)min(bl, nblocks - 1) * 20;

    float acc[MT][8];
    float accm[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        accm[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc[m][j] = 0.0f;
        }
    }
    auto row = [&](uint32_t dm, uint32_t x, const float (&a)[MT]) {
        const float d = h2f(dm & 0xffffu);
        const float mn = h2f(dm >> 16);
        const uint32_t lo = x & 0x0f0f0f0fu, hi = (x >> 4) & 0x0f0f0f0fu;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float ad = a[m] * d;
            accm[m] = fmaf(a[m], mn, accm[m]);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                acc[m][b] = fmaf(ad, (float)((lo >> (8 * b)) & 0xffu), acc[m][b]);
                acc[m][4 + b] = fmaf(ad, (float)((hi >> (8 * b)) & 0xffu), acc[m][4 + b]);
            }
        }
    };
    using AT = std::conditional_t<AF16, _Float16, float>;
    if constexpr (SOA) {
        // the k-blocked nibble plane: per group of 8 rows a lane's dword of
        // its block is 32 contiguous bytes (two 16-byte loads); wave w takes
        // groups w, w + 4, ..., U / 8 groups per batch, rows past k1 masked
        constexpr int GB = U / 8;
        const int bc = min(bl, nblocks - 1);
        for (int g0 = k0 / 8 + wave; 8 * g0 < k1; g0 += 4 * GB) {
            v4i xq[GB][2];
            uint32_t dmw[GB][8];
            AT ar[GB][8][MT];
#pragma unroll
            for (int gg = 0; gg < GB; ++gg) {
                const int64_t grp = min(g0 + 4 * gg, (k1 - 1) / 8);
                const v4i* xs = reinterpret_cast<const v4i*>(soa_group(p, bc, 8 * grp) + jq * 32);
                xq[gg][0] = xs[0];
                xq[gg][1] = xs[1];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int64_t r = 8 * grp + e < k1 ? 8 * grp + e : k1 - 1;
                    dmw[gg][e] = soa_dm(p, bc, r);
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        ar[gg][e][m] = static_cast<const AT*>(p.a)[(int64_t)min(m, p.m - 1) * p.lda + r];
                    }
                }
            }
            // keep the scheduler from sinking the loads into the arithmetic
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int gg = 0; gg < GB; ++gg) {
                const uint32_t xv[8] = {(uint32_t)xq[gg][0].x, (uint32_t)xq[gg][0].y, (uint32_t)xq[gg][0].z,
                                        (uint32_t)xq[gg][0].w, (uint32_t)xq[gg][1].x, (uint32_t)xq[gg][1].y,
                                        (uint32_t)xq[gg][1].z, (uint32_t)xq[gg][1].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int r = 8 * (g0 + 4 * gg) + e;
                    float a[MT];
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        a[m] = (m < p.m && r < k1) ? (float)ar[gg][e][m] : 0.0f;
                    }
                    row(dmw[gg][e], xv[e], a);
                }
            }
        }
    } else {
    // whole batches of U rows, the ones past k1 masked (their A value is 0
    // and their address clamped), so a wave waits on memory once per batch
    for (int k = k0 + wave; k < k1; k += 4 * U) {
        uint32_t dm[U], x[U];
        AT ar[U][MT];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kr = k + 4 * u;
            const uint8_t* src = col + (int64_t)min(kr, k1 - 1) * p.ldb;
            dm[u] = *reinterpret_cast<const uint32_t*>(src);
            x[u] = *reinterpret_cast<const uint32_t*>(src + 4 + 4 * jq);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                // unconditional load (clamped row and column), masked below:
                // a branch or a use here would split the batch
                ar[u][m] = static_cast<const AT*>(p.a)[(int64_t)min(m, p.m - 1) * p.lda + min(kr, k1 - 1)];
            }
        }
        // keep the scheduler from sinking the loads into the arithmetic
        // below (it would otherwise keep only two rows in flight)
        __builtin_amdgcn_sched_barrier(0);
        float a[U][MT];
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                a[u][m] = (m < p.m && k + 4 * u < k1) ? (float)ar[u][m] : 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            row(dm[u], x[u], a[u]);
        }
    }
    }
    if (wave > 0) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                red[wave - 1][m][j][lane] = acc[m][j] + accm[m];
            }
        }
    }
    __syncthreads();
    if (wave != 0 || !live) {
        return;
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        if (m >= p.m) {
            continue;
        }
        float* dst = p.partial + ((int64_t)split * p.m + m) * p.n + bl * 32 + 4 * jq;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int n = bl * 32 + 4 * jq + (j & 3) + 16 * (j >> 2);
            const float v = acc[m][j] + accm[m] + red[0][m][j][lane] + red[1][m][j][lane] + red[2][m][j][lane];
            if (n < p.n) {
                dst[(j & 3) + 16 * (j >> 2)] = v;
            }
        }
    }
}

// Sum of the K-split partials: TPG threads per output element, each summing
// every TPG-th split with four loads in flight, combined by a fixed shuffle
// tree (the same order on every run).
template <int TPG>
__global__ __launch_bounds__(256) void reduce_q4_1(Q41Kern p)
{
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) / TPG;
    const int j = threadIdx.x % TPG;
    const int64_t total = (int64_t)p.m * p.n;
    const bool in = i < total;
    const float* src = p.partial + (in ? i : 0);
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    if (in) {
        int sp = j;
        for (; sp + 3 * TPG < p.splits; sp += 4 * TPG) {
            s0 += src[(int64_t)sp * total];
            s1 += src[(int64_t)(sp + TPG) * total];
            s2 += src[(int64_t)(sp + 2 * TPG) * total];
            s3 += src[(int64_t)(sp + 3 * TPG) * total];
        }
        for (; sp < p.splits; sp += TPG) {
            s0 += src[(int64_t)sp * total];
        }
    }
    float s = (s0 + s1) + (s2 + s3);
#pragma unroll
    for (int off = 1; off < TPG; off <<= 1) {
        s += __shfl_xor(s, off, TPG);
    }
    if (!in || j != 0) {
        return;
    }
    const int m = (int)(i / p.n);
    const int n = (int)(i - (int64_t)m * p.n);
    store_out(p, m, n, s);
}

// ---------------------------------------------------------------------------
// GEMV, blocks along N, one launch: gemv_q4_1_kn_dma.
//
// A workgroup owns one column group of 32 blocks (1024 columns; 640 bytes of
// every row, whole 128-byte lines when the row pitch is a multiple of 128) and
// a range of kper rows (a multiple of 32). Its rows reach LDS by DMA, 32 rows
// (20 KiB) per stage, NS stages in flight. Lane (h, b, jq) owns nibble dword jq
// of block b (columns 32b + 4jq + j and 32b + 16 + 4jq + j, j < 4) for the row
// pairs h, h + W/2, ... of each stage (W waves, two per class). Per row pair
// (k, k+1):
//   s = (a_k, a_k+1) * (d_k, d_k+1) = sv + sl   v_pk_mul_f16, then v_pk_fma_f16
//                                               for the exact rounding error sl
//   t = (byte j of x_k, 0, byte j of x_k+1, 0)  one v_perm per j
//   lo = t & 0x000f000f | 0x54005400 = (64 + q/16) pairs, dotted with 16 sv, 16 sl
//   hi = t & 0x00f000f0 | 0x54005400 = (64 + q) pairs, dotted with sv, sl
// so lo sums 1024 S + sum s q and hi 64 S + sum s q, S = sum s (kept per stage
// and removed when the stage's sums are folded into the totals, so the offset
// never grows beyond one stage), plus sum a m per block from (a) . (m) pairs.
// Products of f16 pairs are exact in the f32 dot, so the only rounding is the
// f32 accumulation (sv alone would cost 2^-11 of every a d term).
// The K splits of a column group meet at the end: each stores its 1024 sums
// per row of A (device-coherent sc1 stores), then its flag (the launch epoch);
// a workgroup that then reads every split's flag set sums the splits in split
// order (deterministic) and writes C -- the last to arrive always does, and
// another that reads the flags at the same moment writes the same bits. The
// summing workgroup clears the flags, so a replayed graph (same epoch) finds
// them clear; a flag word left by anything else is not this launch's epoch.
// ---------------------------------------------------------------------------
constexpr int kKnCB = 32;                   // blocks per column group
constexpr int kKnGroupBytes = kKnCB * 20;   // 640 bytes of each row
constexpr int kKnRS = 32;                   // rows per stage
constexpr int kKnStage = kKnRS * kKnGroupBytes;   // 20 KiB = 20 DMA instructions of 1 KiB
constexpr int kKnNS = 4;                    // stages in flight

struct KnDma {
    int splits, kper;       // splits <= 64
    float* part;            // [groups][splits][MT][1024]
    uint64_t* flag;         // [groups][splits]: the epoch once a split's partials are out, else 0
    uint64_t epoch;         // unique per launch (graph replays repeat it), never 0
};

template <int MT, int W>
__global__ __launch_bounds__(W * 64) void gemv_q4_1_kn_dma(Q41Kern p, KnDma kd)
{
    // the ring alone (two workgroups per CU fit in LDS); the end-of-kernel
    // reduction and the ticket reuse its first bytes
    __shared__ __attribute__((aligned(1024))) uint8_t ring[kKnNS * kKnStage];
    int* s_last = reinterpret_cast<int*>(ring + kKnStage);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int cg = blockIdx.x;
    const int sp = blockIdx.y;
    const int k0 = sp * kd.kper;
    const int k1 = min(p.k, k0 + kd.kper);
    const int stages = (k1 - k0 + kKnRS - 1) / kKnRS;
    const QBufRsrc rs = q_buffer_rsrc(p.b + (int64_t)k0 * p.ldb + (int64_t)cg * kKnGroupBytes, 0x7fffffffu);
    // DMA: chunk c = wave + W q of a stage (20 of 1 KiB) is 64 16-byte pieces;
    // piece i of the stage is row i / 40, bytes 16 (i % 40) .. +15 of the
    // row's 640. Pieces past the end of a row (a last, narrower column group)
    // re-read its last piece, and rows past K re-read row K - 1, so no load
    // leaves the weight; those columns and rows are never used.
    const int valid16 = (int)min<int64_t>(kKnGroupBytes, p.ldb - (int64_t)cg * kKnGroupBytes) / 16;
    constexpr int NQ = (20 + W - 1) / W;        // DMA instructions per wave and stage (at most)
    const int nq = (20 - wave + W - 1) / W;     // this wave's
    int prow[NQ], pcol[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int i = (wave + W * q) * 64 + lane;
        prow[q] = i / 40;
        pcol[q] = min(i % 40, valid16 - 1) * 16;
    }
    auto issue = [&](int st) {
        uint8_t* dst = ring + (st % kKnNS) * kKnStage;
        const int rmax = p.k - 1 - (k0 + st * kKnRS);
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            if (q < nq) {
                q_buffer_load_lds16<2>(rs, dst + (wave + W * q) * 1024, min(prow[q], rmax) * (int)p.ldb + pcol[q],
                                    st * kKnRS * (int)p.ldb);
            }
        }
    };
#pragma unroll
    for (int st = 0; st < kKnNS; ++st) {
        if (st < stages) {
            issue(st);
        }
    }

    constexpr int H = W / 2;                // row-pair classes: h takes pairs h, h + H, ...
    const int h = wave >> 1;
    const int b = (tid >> 2) & 31;          // block in the group
    const int jq = tid & 3;                 // nibble dword of the block
    const v2h sixteen = {(_Float16)16.0f, (_Float16)16.0f};
    const v2h ones = {(_Float16)1.0f, (_Float16)1.0f};
    float tot_lo[MT][4], tot_hi[MT][4], tot_m[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        tot_m[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            tot_lo[m][j] = 0.0f;
            tot_hi[m][j] = 0.0f;
        }
    }
    // A through the scalar cache (constant address space: A is not written
    // here), so its loads stay out of vmcnt, which counts the ring's DMA
    typedef const __attribute__((address_space(4))) uint32_t* ConstU32;
    ConstU32 a32[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        a32[m] = (ConstU32)(static_cast<const _Float16*>(p.a) + (int64_t)min(m, p.m - 1) * p.lda);
    }
    for (int st = 0; st < stages; ++st) {
        // stage st landed (the later ones may be in flight), in every wave
        if (st + kKnNS <= stages) {
            if (nq == NQ) {
                wait_vmcnt<(kKnNS - 1) * NQ>();
            } else {
                wait_vmcnt<(kKnNS - 1) * (NQ - 1)>();
            }
        } else {
            wait_vmcnt<0>();
        }
        q_block_barrier();
        const uint8_t* sb = ring + (st % kKnNS) * kKnStage;
        float acc_lo[MT][4], acc_hi[MT][4], sum_s[MT], acc_m[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            sum_s[m] = 0.0f;
            acc_m[m] = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc_lo[m][j] = 0.0f;
                acc_hi[m][j] = 0.0f;
            }
        }
        // this wave's (a_k, a_k+1) words of the stage, loaded together; rows
        // past this split's range (K and k1 are even) and rows of A past M are 0
        constexpr int RPL = kKnRS / 2 / H;   // row pairs per lane and stage
        uint32_t aws[MT][RPL];
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            const int kr = k0 + st * kKnRS + 2 * (H * i + h);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                aws[m][i] = a32[m][min(kr, p.k - 2) >> 1];
            }
        }
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            const int kr = k0 + st * kKnRS + 2 * (H * i + h);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                aws[m][i] = (m < p.m && kr < k1) ? aws[m][i] : 0u;
            }
        }
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            const int rp = H * i + h;                       // row pair within the stage
            const uint8_t* r0 = sb + 2 * rp * kKnGroupBytes + b * 20;
            const uint32_t dm0 = *reinterpret_cast<const uint32_t*>(r0);
            const uint32_t dm1 = *reinterpret_cast<const uint32_t*>(r0 + kKnGroupBytes);
            const uint32_t x0 = *reinterpret_cast<const uint32_t*>(r0 + 4 + 4 * jq);
            const uint32_t x1 = *reinterpret_cast<const uint32_t*>(r0 + kKnGroupBytes + 4 + 4 * jq);
            // (d_k, d_k+1) and (m_k, m_k+1) as f16 pairs
            const v2h d2 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(dm1, dm0, 0x05040100u));
            const v2h m2 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(dm1, dm0, 0x07060302u));
            // s = a d as an unevaluated f16 sum sv + sl: sv the rounded
            // product, sl = fma(a, d, -sv) its exact rounding error
            v2h sv[MT], sl[MT], s16[MT], sl16[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const v2h a2 = __builtin_bit_cast(v2h, aws[m][i]);
                sv[m] = a2 * d2;
                sl[m] = __builtin_elementwise_fma(a2, d2, -sv[m]);
                s16[m] = sv[m] * sixteen;
                sl16[m] = sl[m] * sixteen;
                sum_s[m] = __builtin_amdgcn_fdot2(sv[m], ones, sum_s[m], false);
                sum_s[m] = __builtin_amdgcn_fdot2(sl[m], ones, sum_s[m], false);
                acc_m[m] = __builtin_amdgcn_fdot2(a2, m2, acc_m[m], false);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // (byte j of x0, 0, byte j of x1, 0): selector 0x0c is a zero byte
                const uint32_t sel = 0x0c000c00u | (uint32_t)(4 + j) << 16 | (uint32_t)j;
                const uint32_t t = __builtin_amdgcn_perm(x1, x0, sel);
                const v2h lo = __builtin_bit_cast(v2h, and_or_u32(t, 0x000f000fu, 0x54005400u));
                const v2h hi = __builtin_bit_cast(v2h, and_or_u32(t, 0x00f000f0u, 0x54005400u));
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    acc_lo[m][j] = __builtin_amdgcn_fdot2(s16[m], lo, acc_lo[m][j], false);
                    acc_lo[m][j] = __builtin_amdgcn_fdot2(sl16[m], lo, acc_lo[m][j], false);
                    acc_hi[m][j] = __builtin_amdgcn_fdot2(sv[m], hi, acc_hi[m][j], false);
                    acc_hi[m][j] = __builtin_amdgcn_fdot2(sl[m], hi, acc_hi[m][j], false);
                }
            }
        }
        // fold the stage: remove the 64 / 1024 offsets while they are small
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            tot_m[m] += acc_m[m];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                tot_lo[m][j] += fmaf(-1024.0f, sum_s[m], acc_lo[m][j]);
                tot_hi[m][j] += fmaf(-64.0f, sum_s[m], acc_hi[m][j]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's reads of the slot returned
        q_block_barrier();                  // every wave is done with this slot
        if (st + kKnNS < stages) {
            issue(st + kKnNS);
        }
    }

    // the row-pair classes meet in LDS (the ring is free now)
    float* red = reinterpret_cast<float*>(ring);      // [H - 1][MT][128 lanes][8]
    if (h > 0) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                red[(((h - 1) * MT + m) * 128 + (tid & 127)) * 8 + j] = tot_lo[m][j] + tot_m[m];
                red[(((h - 1) * MT + m) * 128 + (tid & 127)) * 8 + 4 + j] = tot_hi[m][j] + tot_m[m];
            }
        }
    }
    __syncthreads();
    const QBufRsrc rp = q_buffer_rsrc(reinterpret_cast<char*>(kd.part) + (int64_t)cg * kd.splits * MT * 4096,
                                      0x7fffffffu);
    if (h == 0) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            v4f lo4, hi4;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                lo4[j] = tot_lo[m][j] + tot_m[m];
                hi4[j] = tot_hi[m][j] + tot_m[m];
#pragma unroll
                for (int g = 0; g < H - 1; ++g) {
                    lo4[j] += red[((g * MT + m) * 128 + tid) * 8 + j];
                    hi4[j] += red[((g * MT + m) * 128 + tid) * 8 + 4 + j];
                }
            }
            // columns 32b + 4jq .. +3 and 32b + 16 + 4jq .. +3 of the group
            const int off = (sp * MT + m) * 4096 + (32 * b + 4 * jq) * 4;
            q_buffer_store16_sc1(rp, __builtin_bit_cast(v4i, lo4), off);
            q_buffer_store16_sc1(rp, __builtin_bit_cast(v4i, hi4), off + 64);
        }
    }
    // Publish: once this workgroup's partial stores are complete, its flag
    // (the launch epoch) goes out; then wave 0 reads every split's flag. A
    // workgroup that finds them all set sums the splits: the last to arrive
    // always does, and one that reads the flags at the same moment may too,
    // writing the same bits (the sum runs in split order).
    wait_vmcnt<0>();
    __syncthreads();
    const QBufRsrc rf = q_buffer_rsrc(kd.flag + (int64_t)cg * kd.splits, 0x7fffffffu);
    if (wave == 0) {
        if (lane == 0) {
            q_buffer_store8_sc1(rf, kd.epoch, sp * 8);
        }
        wait_vmcnt<0>();
        const uint64_t f = lane < kd.splits ? q_buffer_load8_sc1(rf, lane * 8) : kd.epoch;
        const bool all = __builtin_amdgcn_ballot_w64(f != kd.epoch) == 0;
        if (lane == 0) {
            *s_last = all;
        }
    }
    __syncthreads();
    if (!*s_last) {
        return;
    }
    // 1024 columns x MT rows: 4 consecutive columns per thread and row
    if constexpr (MT == 1 && W == 8) {
        // one row: two threads per column quad, each summing its half of the
        // splits in split order with every load in flight at once (half 0
        // takes splits 0 .. 15, half 1 the rest), then half 0 adds half 1's sum
        static_assert(kKnNS * kKnStage >= 256 * 16, "the halves meet in the ring");
        const int half = tid >> 8, q = tid & 255;
        const int nq = cg * 1024 + 4 * q;
        const int sa = half ? 16 : 0, sb = half ? kd.splits : min(16, kd.splits);
        v4f sum = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int s0 = sa; s0 < sb; s0 += 16) {
            v4f part[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int s2 = min(s0 + u, sb - 1);
                part[u] = __builtin_bit_cast(v4f, q_buffer_load16_sc1(rp, s2 * MT * 4096 + q * 16));
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                if (s0 + u < sb) {
                    sum += part[u];
                }
            }
        }
        v4f* xs = reinterpret_cast<v4f*>(ring);
        if (half == 1) {
            xs[q] = sum;
        }
        __syncthreads();
        if (half == 0 && nq < p.n) {
            if (kd.splits > 16) {
                sum += xs[q];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (nq + e < p.n) {
                    store_out(p, 0, nq + e, sum[e]);
                }
            }
        }
    } else {
    const int n = cg * 1024 + 4 * tid;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        if (tid >= 256 || m >= p.m || n >= p.n) {
            continue;
        }
        // 16 splits' loads in flight at a time, summed in split order
        v4f sum = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int s0 = 0; s0 < kd.splits; s0 += 16) {
            v4f part[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int s2 = min(s0 + u, kd.splits - 1);
                part[u] = __builtin_bit_cast(v4f, q_buffer_load16_sc1(rp, (s2 * MT + m) * 4096 + tid * 16));
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                if (s0 + u < kd.splits) {
                    sum += part[u];
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (n + e < p.n) {
                store_out(p, m, n + e, sum[e]);
            }
        }
    }
    }
    // clear the flags for the next launch on this workspace (a replayed graph
    // reuses the epoch); every split has published by now
    if (tid < kd.splits) {
        q_buffer_store8_sc1(rf, 0ull, tid * 8);
    }
}

// ---------------------------------------------------------------------------
// GEMV over the prepacked blocks-along-N planes, f16 A, M <= 2 per launch, K
// % 8 == 0: one launch, no workspace. Workgroup j owns block column j (32
// columns) over the whole of K, which the planes hold as two contiguous runs
// (K / 8 groups of 128 nibble bytes, K d|m dwords), so no partial sum leaves
// it. The nibble run is read as consecutive 16-byte chunks by consecutive
// lanes (every wave load is 1 KiB of whole lines: the access pattern that
// streams HBM at full rate; 32-byte pieces per lane ran 40 % slower). Chunk c
// of a group is nibble dword c / 2 (columns 4 (c/2) + i from the low
// nibbles, 16 + 4 (c/2) + i from the high, i < 4) of the group's rows 4 (c %
// 2) .. + 3, so lane t always owns chunk t % 8 of the groups t / 8, t / 8 +
// T / 8, ...; with it the 4 rows' d|m dwords (16 bytes) and A's 4 halves per
// row of A, U chunks in flight. Per row pair (k, k+1) the arithmetic of
// gemv_q4_1_kn_dma: s = (a_k, a_k+1) * (d_k, d_k+1) as the exact f16 sum
// sv + sl, nibble pairs of the two rows widened by v_perm / v_and_or (64 +
// q/16 and 64 + q), dotted with s in f32, the low nibbles' sums scaled by 16
// and the 1024 S and 64 S offsets removed per batch; plus sum a m per block.
// The lanes of a column
// meet in LDS in lane order (deterministic). Bound: HBM.
// ---------------------------------------------------------------------------
template <int MT, int W, int U>
__global__ __launch_bounds__(W * 64) void gemv_q4_1_bcm(Q41Kern p)
{
    constexpr int T = W * 64, NS = T / 4;        // lanes per nibble dword
    __shared__ float red[MT * 32][NS + 1];
    const int t = threadIdx.x;
    const int c = t & 7, jq = c >> 1, h = c & 1;
    const int slot = (t >> 3) * 2 + h;           // the lane among those of its dword
    const int64_t j = blockIdx.x;                // block column
    const int nch = p.k;                         // 16-byte chunks: 8 per group of 8 rows
    const v4i* nib = reinterpret_cast<const v4i*>(p.b + j * p.ldb);
    const uint32_t* dmc = p.bdm + j * p.ldbdm;
    const _Float16* A = static_cast<const _Float16*>(p.a);
    const v2h ones = {(_Float16)1.0f, (_Float16)1.0f};
    float tot_lo[MT][4], tot_hi[MT][4], tot_m[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        tot_m[m] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            tot_lo[m][i] = 0.0f;
            tot_hi[m][i] = 0.0f;
        }
    }
    for (int i0 = t; i0 < nch; i0 += U * T) {
        v4i x[U], dmv[U];
        v2u32 av[U][MT];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // chunk ci: rows r0 .. r0 + 3 (a chunk past K re-reads the last)
            const int ci = min(i0 + u * T, nch - 8 + c);
            const int r0 = (ci >> 3) * 8 + 4 * h;
            x[u] = __builtin_nontemporal_load(nib + ci);
            dmv[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(dmc + r0));
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                av[u][m] = *reinterpret_cast<const v2u32*>(A + (int64_t)min(m, p.m - 1) * p.lda + r0);
            }
        }
        float acc_lo[MT][4], acc_hi[MT][4], sum_s[MT], acc_m[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            sum_s[m] = 0.0f;
            acc_m[m] = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc_lo[m][i] = 0.0f;
                acc_hi[m][i] = 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // a chunk past K (the clamped re-read) and rows of A past M count 0
            const bool live = i0 + u * T < nch;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t x0 = (uint32_t)x[u][2 * e], x1 = (uint32_t)x[u][2 * e + 1];
                const uint32_t dm0 = (uint32_t)dmv[u][2 * e], dm1 = (uint32_t)dmv[u][2 * e + 1];
                const v2h d2 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(dm1, dm0, 0x05040100u));
                const v2h m2 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(dm1, dm0, 0x07060302u));
                v2h sv[MT], sl[MT];
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const uint32_t aw = (live && m < p.m) ? (uint32_t)av[u][m][e] : 0u;
                    const v2h a2 = __builtin_bit_cast(v2h, aw);
                    sv[m] = a2 * d2;
                    sl[m] = __builtin_elementwise_fma(a2, d2, -sv[m]);
                    sum_s[m] = __builtin_amdgcn_fdot2(sv[m], ones, sum_s[m], false);
                    sum_s[m] = __builtin_amdgcn_fdot2(sl[m], ones, sum_s[m], false);
                    acc_m[m] = __builtin_amdgcn_fdot2(a2, m2, acc_m[m], false);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // (byte i of x0, 0, byte i of x1, 0): selector 0x0c is a zero byte
                    const uint32_t sel = 0x0c000c00u | (uint32_t)(4 + i) << 16 | (uint32_t)i;
                    const uint32_t tt = __builtin_amdgcn_perm(x1, x0, sel);
                    const v2h lo = __builtin_bit_cast(v2h, and_or_u32(tt, 0x000f000fu, 0x54005400u));
                    const v2h hi = __builtin_bit_cast(v2h, and_or_u32(tt, 0x00f000f0u, 0x54005400u));
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        acc_lo[m][i] = __builtin_amdgcn_fdot2(sv[m], lo, acc_lo[m][i], false);
                        acc_lo[m][i] = __builtin_amdgcn_fdot2(sl[m], lo, acc_lo[m][i], false);
                        acc_hi[m][i] = __builtin_amdgcn_fdot2(sv[m], hi, acc_hi[m][i], false);
                        acc_hi[m][i] = __builtin_amdgcn_fdot2(sl[m], hi, acc_hi[m][i], false);
                    }
                }
            }
        }
        // fold the batch: remove the 64 S offsets while they are small; the low
        // nibbles' sums (of s (64 + q/16)) are scaled by 16 exactly first
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            tot_m[m] += acc_m[m];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                tot_lo[m][i] += fmaf(-1024.0f, sum_s[m], 16.0f * acc_lo[m][i]);
                tot_hi[m][i] += fmaf(-64.0f, sum_s[m], acc_hi[m][i]);
            }
        }
    }
    // column col of the block, row m: word (m * 32 + col, slot)
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            red[m * 32 + 4 * jq + i][slot] = tot_lo[m][i] + tot_m[m];
            red[m * 32 + 16 + 4 * jq + i][slot] = tot_hi[m][i] + tot_m[m];
        }
    }
    __syncthreads();
    if (t < MT * 32) {
        const int m = t / 32, n = (int)j * 32 + t % 32;
        float v = 0.0f;
#pragma unroll 8
        for (int q = 0; q < NS; ++q) {
            v += red[t][q];
        }
        if (m < p.m && n < p.n) {
            store_out(p, m, n, v);
        }
    }
}


// ---------------------------------------------------------------------------
// Skinny GEMM over the prepacked blocks-along-N planes: f16 A with 3 <= M <=
// 16 rows per launch, K % 256 == 0. Workgroup j owns block column j (32
// columns); its 4 waves take K quarters, each through its own DMA ring in LDS
// (NS stages of 64 k: the 8 nibble groups, 1 KiB; the 64 d|m dwords, 256
// bytes; A's 16 rows x 128 bytes with row r's 16-byte chunk c in slot c ^ ((r
// >> 1) & 7), so the 16 rows a fragment read serves hit 16 bank groups), so a
// wave waits only on its own loads, never at a barrier. Per 32-k slice lane l
// decodes the slice's rows 8 (l / 16) .. + 7 at columns l % 16 (low nibbles)
// and 16 + l % 16 (high nibbles): byte l % 4 of the rows' nibble dword (l %
// 16) / 4 (a 32-byte LDS read that 4 lanes share), 1024 + q by v_and_or_b32
// under exponent byte 0x64, v_pk_add_f16 removes 1024 exactly and
// v_pk_fma_f16 rounds d * q + m once (the f16 weights of the ring GEMMs); then
// two v_mfma_f32_16x16x32_f16 with A's fragment (row l % 16, the same 8 k).
// The quarters meet in LDS in wave order (deterministic). Bound: HBM.
// ---------------------------------------------------------------------------
template <int NS>
__global__ __launch_bounds__(256) void gemv_q4_1_bcm_mfma(Q41Kern p)
{
    constexpr int W = 4;
    constexpr int kNib = 1024, kDm = 256, kAt = 2048, kSt = kNib + kDm + kAt;
    constexpr int L = 4;                              // DMA instructions per stage
    static_assert((NS - 1) * L < 64, "vmcnt range");
    static_assert(W * NS * kSt >= (W - 1) * 2 * 64 * 16, "the quarters' sums fit the ring");
    __shared__ __attribute__((aligned(1024))) uint8_t ring[W * NS * kSt];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t j = blockIdx.x;
    const uint8_t* nib = p.b + j * p.ldb;
    const uint8_t* dmc = reinterpret_cast<const uint8_t*>(p.bdm + j * p.ldbdm);
    const _Float16* A = static_cast<const _Float16*>(p.a);
    const int kq = p.k / W;
    const int kbeg = wave * kq;
    const int nst = kq / 64;
    uint8_t* my = ring + wave * NS * kSt;
    // A rows staged by lane: instruction q holds rows 8 q .. 8 q + 7
    const _Float16* a_src[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int r = 8 * q + (lane >> 3);
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        a_src[q] = A + (int64_t)min(r, p.m - 1) * p.lda + kbeg + 8 * c;
    }
    auto issue = [&](int st) {
        uint8_t* base = my + (st % NS) * kSt;
        const int k0 = kbeg + 64 * st;
        __builtin_amdgcn_global_load_lds(NNOPS_GPTR(nib + (int64_t)(k0 / 8) * 128 + 16 * lane), NNOPS_LPTR(base), 16,
                                         0, 2);
        if (lane < 16) {
            __builtin_amdgcn_global_load_lds(NNOPS_GPTR(dmc + (int64_t)k0 * 4 + 16 * lane),
                                             NNOPS_LPTR(base + kNib), 16, 0, 2);
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            __builtin_amdgcn_global_load_lds(NNOPS_GPTR(a_src[q] + 64 * st), NNOPS_LPTR(base + kNib + kDm + 1024 * q),
                                             16, 0, 0);
        }
    };
#pragma unroll
    for (int st = 0; st < NS - 1; ++st) {
        if (st < nst) {
            issue(st);
        }
    }
    const int ar = lane & 15, g = lane >> 4;          // A row; k group of the slice
    const int col = lane & 15;
    const uint32_t sel = 0x0c000c00u | (uint32_t)(4 + (col & 3)) << 16 | (uint32_t)(col & 3);
    v4f acc0 = v4f{0.0f, 0.0f, 0.0f, 0.0f}, acc1 = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const v2h k1024 = __builtin_bit_cast(v2h, 0x64006400u);
    for (int st = 0; st < nst; ++st) {
        if (st + NS - 1 < nst) {
            issue(st + NS - 1);
            wait_vmcnt<(NS - 1) * L>();
        } else {
            wait_vmcnt<0>();
        }
        asm volatile("" ::: "memory");
        const uint8_t* base = my + (st % NS) * kSt;
#pragma unroll
        for (int sl = 0; sl < 2; ++sl) {
            const int cf = 4 * sl + g;                    // A chunk of the lane's 8 k
            const v8h af = *reinterpret_cast<const v8h*>(base + kNib + kDm + ar * 128 + ((cf ^ ((ar >> 1) & 7)) << 4));
            const uint8_t* gp = base + (4 * sl + g) * 128 + 32 * (col >> 2);
            const v4i n0 = *reinterpret_cast<const v4i*>(gp);
            const v4i n1 = *reinterpret_cast<const v4i*>(gp + 16);
            const uint8_t* dp = base + kNib + (32 * sl + 8 * g) * 4;
            const v4i d0 = *reinterpret_cast<const v4i*>(dp);
            const v4i d1 = *reinterpret_cast<const v4i*>(dp + 16);
            const uint32_t nw[8] = {(uint32_t)n0.x, (uint32_t)n0.y, (uint32_t)n0.z, (uint32_t)n0.w,
                                    (uint32_t)n1.x, (uint32_t)n1.y, (uint32_t)n1.z, (uint32_t)n1.w};
            const uint32_t dw[8] = {(uint32_t)d0.x, (uint32_t)d0.y, (uint32_t)d0.z, (uint32_t)d0.w,
                                    (uint32_t)d1.x, (uint32_t)d1.y, (uint32_t)d1.z, (uint32_t)d1.w};
            uint32_t wl[4], wh[4];
#pragma unroll
            for (int rp = 0; rp < 4; ++rp) {
                const uint32_t t = __builtin_amdgcn_perm(nw[2 * rp + 1], nw[2 * rp], sel);
                const v2h ql = __builtin_bit_cast(v2h, and_or_u32(t, 0x000f000fu, 0x64006400u)) - k1024;
                const v2h qh = __builtin_bit_cast(v2h, and_or_u32(t >> 4, 0x000f000fu, 0x64006400u)) - k1024;
                const v2h d2 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(dw[2 * rp + 1], dw[2 * rp], 0x05040100u));
                const v2h m2 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(dw[2 * rp + 1], dw[2 * rp], 0x07060302u));
                wl[rp] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(ql, d2, m2));
                wh[rp] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(qh, d2, m2));
            }
            const v8h bl = __builtin_bit_cast(v8h, v4i{(int)wl[0], (int)wl[1], (int)wl[2], (int)wl[3]});
            const v8h bh = __builtin_bit_cast(v8h, v4i{(int)wh[0], (int)wh[1], (int)wh[2], (int)wh[3]});
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bl, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bh, acc1, 0, 0, 0);
        }
    }
    // the quarters meet in wave order: rows 4 (lane / 16) + r of columns
    // lane % 16 (acc0) and 16 + lane % 16 (acc1)
    __syncthreads();
    v4f* red = reinterpret_cast<v4f*>(ring);
    if (wave > 0) {
        red[((wave - 1) * 2 + 0) * 64 + lane] = acc0;
        red[((wave - 1) * 2 + 1) * 64 + lane] = acc1;
    }
    __syncthreads();
    if (wave != 0) {
        return;
    }
#pragma unroll
    for (int w = 0; w < W - 1; ++w) {
        acc0 += red[(w * 2 + 0) * 64 + lane];
        acc1 += red[(w * 2 + 1) * 64 + lane];
    }
    const int n = (int)j * 32 + col;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = 4 * g + r;
        if (m < p.m) {
            if (n < p.n) {
                store_out(p, m, n, acc0[r]);
            }
            if (n + 16 < p.n) {
                store_out(p, m, n + 16, acc1[r]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Skinny GEMM, blocks along K ([N][K/32]), f16 A with 3 <= M <= 16 rows per
// launch (more rows: one launch per 16), K % 256 == 0: the weight streams
// once, its blocks decoded to f16 and multiplied on the matrix cores.
//
// A workgroup of 2 x KH waves owns 32 weight rows: wave w takes the 16 rows
// 16 (w % 2) .. and the K part w / 2 of KH. Each part runs in stages of 8
// blocks (256 k), NS stages in flight; a stage is, per part, DMA regions in
// LDS:
//   weights  per wave 16 rows x 176 bytes: the rows' 160 stage bytes (10
//            16-byte chunks) plus a pad chunk, so the 16 rows a read serves
//            fall on 16 distinct bank groups (176 bytes = 44 dwords per row);
//   A        16 rows x 528 bytes, shared by the part's two waves: the stage's
//            256 halves plus a pad chunk (132 dwords per row: a 16-byte read
//            per row of 16 rows covers the 64 banks once).
// The pads come from the DMA itself: lane i of piece q writes 16 bytes at
// q * 1024 + 16 i, so chunk c = 64 q + i is given row c / 11, column c % 11
// (c / 33, c % 33 for A), and a pad or surplus chunk re-reads a valid one.
// Each wave issues its rows and half of its part's A pieces; a stage is read
// after every wave has waited for its own pieces and passed the block
// barrier. Per block, lane l decodes the 8 values of row l % 16 at k = 8 (l /
// 16) .. + 7 (low or high nibbles of bytes 0-7 or 8-15): a byte permute and
// v_and_or_b32 make (1024 + q) f16 pairs, v_pk_add_f16 removes 1024 exactly
// and v_pk_fma_f16 rounds d * q + m once; the 16 x 32 weight tile and A's
// 32 x 16 tile (lane l: row l % 16, the same 8 k) meet in one
// v_mfma_f32_16x16x32_f16. The K parts meet in LDS at the end, in part
// order. Bound: the decode at a few waves per SIMD, then HBM.
// ---------------------------------------------------------------------------
constexpr int kSkRows = 32;                          // per workgroup (16 per wave)
constexpr int kSkWChunks = 11;                       // per weight row: 10 + pad
constexpr int kSkWPieces = (16 * kSkWChunks + 63) / 64;        // 3 per wave
constexpr int kSkAChunks = 33;                       // per row of A: 32 + pad
constexpr int kSkAPieces = 10;                       // 16 x 33 = 528 chunks, in 2 x 5 pieces
constexpr int kSkL = kSkWPieces + kSkAPieces / 2;    // DMA instructions per wave and stage

template <int NS, int KH>
__global__ __launch_bounds__(128 * KH) void gemv_q4_1_skinny(Q41Kern p)
{
    static_assert(NS >= 2 && (NS - 2) * kSkL < 64, "vmcnt range");
    constexpr int kAAt = 2 * KH * kSkWPieces * 1024;            // A regions after every wave's rows
    constexpr int kStage = kAAt + KH * kSkAPieces * 1024;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[NS * kStage];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = wave & 1, part = wave >> 1;
    const int n0 = blockIdx.x * kSkRows + 16 * grp;
    const int rows = max(1, min(16, p.n - n0));      // a group past N re-reads row N - 1 (never stored)
    const int stages = p.k / 256 / KH;               // per part (host-checked: K % (256 KH) == 0)
    const int s0 = part * stages;                    // the part's first stage of K
    const QBufRsrc rw = q_buffer_rsrc(p.b + (int64_t)min(n0, p.n - 1) * p.ldb, (uint32_t)((int64_t)rows * p.ldb));
    const QBufRsrc ra = q_buffer_rsrc(p.a, 0x7fffffffu);
    int w_off[kSkWPieces], a_off[kSkAPieces / 2];
#pragma unroll
    for (int q = 0; q < kSkWPieces; ++q) {
        const int c = 64 * q + lane, r = c / kSkWChunks, cc = c % kSkWChunks;
        w_off[q] = (r < 16 && cc < 10) ? min(r, rows - 1) * (int)p.ldb + 16 * cc : 0;
    }
#pragma unroll
    for (int q = 0; q < kSkAPieces / 2; ++q) {
        const int c = 64 * (q + grp * (kSkAPieces / 2)) + lane, m = c / kSkAChunks, cc = c % kSkAChunks;
        a_off[q] = (m < 16 && cc < 32) ? min(m, p.m - 1) * (int)p.lda * 2 + 16 * cc : 0;
    }
    uint8_t* const a_region = ring + kAAt + part * kSkAPieces * 1024;
    auto issue = [&](int s) {
        uint8_t* dst = ring + (s % NS) * kStage;
        const int sg = s0 + s;
#pragma unroll
        for (int q = 0; q < kSkWPieces; ++q) {
            q_buffer_load_lds16<2>(rw, dst + (wave * kSkWPieces + q) * 1024, w_off[q], sg * 160);
        }
#pragma unroll
        for (int q = 0; q < kSkAPieces / 2; ++q) {
            q_buffer_load_lds16(ra, a_region - ring + dst + (grp * (kSkAPieces / 2) + q) * 1024, a_off[q],
                                sg * 512);
        }
    };
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) {
        if (s < stages) {
            issue(s);
        }
    }
    const int r16 = lane & 15, qk = lane >> 4;
    const int nb = 8 * (qk & 1);                     // first nibble byte of this lane's 8 values
    const int sh = 4 * (qk >> 1);                    // low (0) or high (4) nibbles
    const v2h k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = 0; s < stages; ++s) {
        // this wave's pieces of stage s have landed (later stages may be in
        // flight), every wave's reads of stage s - 1 are done, then the barrier
        if (s + NS - 2 < stages) {
            wait_vmcnt<(NS - 2) * kSkL>();
        } else {
            wait_vmcnt<0>();
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);          // lgkmcnt(0)
        q_block_barrier();
        if (s + NS - 1 < stages) {
            issue(s + NS - 1);                       // into the slot of stage s - 1
        }
        const uint8_t* st = ring + (s % NS) * kStage;
        const uint8_t* abase = a_region - ring + st + r16 * (16 * kSkAChunks) + 16 * qk;
        const uint8_t* wbase = st + wave * kSkWPieces * 1024 + r16 * (16 * kSkWChunks);
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const v8h bf = *reinterpret_cast<const v8h*>(abase + 64 * jj);
            const uint8_t* wr = wbase + 20 * jj;
            const uint32_t dm = *reinterpret_cast<const uint32_t*>(wr);
            const uint32_t x0 = *reinterpret_cast<const uint32_t*>(wr + 4 + nb) >> sh;
            const uint32_t x1 = *reinterpret_cast<const uint32_t*>(wr + 8 + nb) >> sh;
            const v2h d2 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(dm, dm, 0x01000100u));
            const v2h m2 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(dm, dm, 0x03020302u));
            uint32_t w[4];
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                // bytes 2h and 2h + 1 of the 8 into the two halves' low bytes
                const uint32_t src = h < 2 ? x0 : x1;
                const uint32_t t = __builtin_amdgcn_perm(src, src, h % 2 == 0 ? 0x0c010c00u : 0x0c030c02u);
                const v2h qv = __builtin_bit_cast(v2h, and_or_u32(t, 0x000f000fu, 0x64006400u)) - k1024;
                w[h] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(d2, qv, m2));
            }
            const v8h af = __builtin_bit_cast(v8h, v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]});
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf, acc, 0, 0, 0);
        }
    }
    if constexpr (KH > 1) {
        // the later K parts hand their sums to part 0 through LDS (the ring is free)
        __builtin_amdgcn_s_waitcnt(0xc07f);
        q_block_barrier();
        v4f* xs = reinterpret_cast<v4f*>(ring);      // [KH - 1][2 groups][64 lanes]
        if (part > 0) {
            xs[((part - 1) * 2 + grp) * 64 + lane] = acc;
        }
        __syncthreads();
        if (part > 0) {
            return;
        }
#pragma unroll
        for (int h = 1; h < KH; ++h) {
            acc += xs[((h - 1) * 2 + grp) * 64 + lane];
        }
    }
    // lane l: rows 4 (l / 16) .. + 3 of the group's 16, column (row of A) l % 16
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int n = n0 + 4 * qk + r;
        if (r16 < p.m && n < p.n) {
            store_out(p, r16, n, acc[r]);
        }
    }
}

// ---------------------------------------------------------------------------
// The skinny GEMM for f32 A (nnops computes f32 x Q4_1 in f32): the same
// workgroup of two waves over 32 weight rows and 256-k stages, the same
// padded weight rows; A's stage is 16 rows x 1040 bytes (256 floats plus a
// pad chunk: 260 dwords per row, so a 16-byte read per row of 16 rows covers
// the 64 banks once). Lane l decodes the 8 values of row l % 16 at k = 8 (l
// / 16) + t to f32 (fmaf(d, q, m), nnops' f32 decode) and runs 8
// v_mfma_f32_16x16x4f32, t = 0 .. 7, against A's same 8 k.
// ---------------------------------------------------------------------------
constexpr int kSkFAChunks = 65;                      // per row of A: 64 + pad
constexpr int kSkFAPieces = 18;                      // 16 x 65 = 1040 chunks, in 2 x 9 pieces
constexpr int kSkFL = kSkWPieces + kSkFAPieces / 2;

template <int NS>
__global__ __launch_bounds__(128) void gemv_q4_1_skinny_f32(Q41Kern p)
{
    static_assert(NS >= 2 && (NS - 2) * kSkFL < 64, "vmcnt range");
    constexpr int kAAt = 2 * kSkWPieces * 1024;
    constexpr int kStage = kAAt + kSkFAPieces * 1024;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[NS * kStage];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * kSkRows + 16 * wave;
    const int rows = max(1, min(16, p.n - n0));      // a group past N re-reads row N - 1 (never stored)
    const int stages = p.k / 256;
    const QBufRsrc rw = q_buffer_rsrc(p.b + (int64_t)min(n0, p.n - 1) * p.ldb, (uint32_t)((int64_t)rows * p.ldb));
    const QBufRsrc ra = q_buffer_rsrc(p.a, 0x7fffffffu);
    int w_off[kSkWPieces], a_off[kSkFAPieces / 2];
#pragma unroll
    for (int q = 0; q < kSkWPieces; ++q) {
        const int c = 64 * q + lane, r = c / kSkWChunks, cc = c % kSkWChunks;
        w_off[q] = (r < 16 && cc < 10) ? min(r, rows - 1) * (int)p.ldb + 16 * cc : 0;
    }
#pragma unroll
    for (int q = 0; q < kSkFAPieces / 2; ++q) {
        const int c = 64 * (q + wave * (kSkFAPieces / 2)) + lane, m = c / kSkFAChunks, cc = c % kSkFAChunks;
        a_off[q] = (m < 16 && cc < 64) ? min(m, p.m - 1) * (int)p.lda * 4 + 16 * cc : 0;
    }
    auto issue = [&](int s) {
        uint8_t* dst = ring + (s % NS) * kStage;
#pragma unroll
        for (int q = 0; q < kSkWPieces; ++q) {
            q_buffer_load_lds16(rw, dst + (wave * kSkWPieces + q) * 1024, w_off[q], s * 160);
        }
#pragma unroll
        for (int q = 0; q < kSkFAPieces / 2; ++q) {
            q_buffer_load_lds16(ra, dst + kAAt + (wave * (kSkFAPieces / 2) + q) * 1024, a_off[q], s * 1024);
        }
    };
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) {
        if (s < stages) {
            issue(s);
        }
    }
    const int r16 = lane & 15, qk = lane >> 4;
    const int nb = 8 * (qk & 1);                     // first nibble byte of this lane's 8 values
    const int sh = 4 * (qk >> 1);                    // low (0) or high (4) nibbles
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = 0; s < stages; ++s) {
        if (s + NS - 2 < stages) {
            wait_vmcnt<(NS - 2) * kSkFL>();
        } else {
            wait_vmcnt<0>();
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);          // lgkmcnt(0)
        q_block_barrier();
        if (s + NS - 1 < stages) {
            issue(s + NS - 1);                       // into the slot of stage s - 1
        }
        const uint8_t* st = ring + (s % NS) * kStage;
        const uint8_t* abase = st + kAAt + r16 * (16 * kSkFAChunks) + 32 * qk;
        const uint8_t* wbase = st + wave * kSkWPieces * 1024 + r16 * (16 * kSkWChunks);
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const v4f a0 = *reinterpret_cast<const v4f*>(abase + 128 * jj);
            const v4f a1 = *reinterpret_cast<const v4f*>(abase + 128 * jj + 16);
            const uint8_t* wr = wbase + 20 * jj;
            const uint32_t dm = *reinterpret_cast<const uint32_t*>(wr);
            const uint32_t x0 = (*reinterpret_cast<const uint32_t*>(wr + 4 + nb) >> sh) & 0x0f0f0f0fu;
            const uint32_t x1 = (*reinterpret_cast<const uint32_t*>(wr + 8 + nb) >> sh) & 0x0f0f0f0fu;
            const float d = h2f(dm & 0xffffu), mn = h2f(dm >> 16);
            float w[8];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                w[b] = fmaf(d, (float)((x0 >> (8 * b)) & 0xffu), mn);
                w[4 + b] = fmaf(d, (float)((x1 >> (8 * b)) & 0xffu), mn);
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w[t], a0[t], acc, 0, 0, 0);
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w[4 + t], a1[t], acc, 0, 0, 0);
            }
        }
    }
    // lane l: rows 4 (l / 16) .. + 3 of the group's 16, column (row of A) l % 16
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int n = n0 + 4 * qk + r;
        if (r16 < p.m && n < p.n) {
            store_out(p, r16, n, acc[r]);
        }
    }
}

// ---------------------------------------------------------------------------
// MFMA GEMM, f16 A.
// ---------------------------------------------------------------------------
constexpr int kQBK = 64;                 // k values per stage (2 Q4_1 blocks)
constexpr int kQLdsRow = kQBK * 2 + 16;  // bytes: 64 halves + 16 pad

// Decode one block (raw: d|m, then 4 dwords of nibbles) to 32 f16 values.
__device__ __forceinline__ void decode_block_f16(const uint32_t raw[5], _Float16 out[32])
{
    const float d = h2f(raw[0] & 0xffffu);
    const float mn = h2f(raw[0] >> 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t q = raw[1 + i];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            out[4 * i + b] = (_Float16)fmaf(d, (float)((q >> (8 * b)) & 15u), mn);
            out[16 + 4 * i + b] = (_Float16)fmaf(d, (float)((q >> (8 * b + 4)) & 15u), mn);
        }
    }
}

template <int BM, int BN, int WM, int WN, bool TRANS_B, bool SOA = false>
__global__ __launch_bounds__(WM * WN * 64, 1) void gemm_q4_1_mfma(Q41Kern p)
{
    constexpr int T = WM * WN * 64;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int CA = BM * (kQBK * 2 / 16) / T;    // 16-byte A chunks per thread
    // B: TRANS_B -> BN rows x 2 blocks; else 64 k rows x BN/32 blocks.
    constexpr int NBLK = TRANS_B ? BN * 2 : kQBK * (BN / 32);
    constexpr int CB = NBLK / T;
    static_assert(CA >= 1 && CB >= 1 && CA * T * 16 == BM * kQBK * 2 && CB * T == NBLK, "tile");

    __shared__ __attribute__((aligned(16))) uint8_t lds_a[2][BM * kQLdsRow];
    __shared__ __attribute__((aligned(16))) uint8_t lds_b[2][BN * kQLdsRow];

    const int tiles_n = (p.n + BN - 1) / BN;
    const int tm = blockIdx.x / tiles_n;
    const int tn = blockIdx.x - tm * tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave / WN) * TM, wn0 = (wave % WN) * TN;
    const int nbk = (p.k + 31) / 32;     // blocks along K (TRANS_B)
    const int nbn = (p.n + 31) / 32;     // blocks along N (!TRANS_B)
    const _Float16* A = static_cast<const _Float16*>(p.a);

    v4i ra[CA];
    uint32_t rb[CB][5];
    auto load_stage = [&](int k0) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int idx = tid + i * T;
            const int r = idx >> 3, c = idx & 7;       // 8 chunks of 8 halves per row
            const int m = min(m0 + r, p.m - 1);
            const int k = k0 + c * 8;
            const _Float16* src = A + (int64_t)m * p.lda + k;
            if (k + 8 <= p.k && ((p.lda & 7) == 0) && (((uintptr_t)A & 15) == 0)) {
                ra[i] = *reinterpret_cast<const v4i*>(src);
            } else {
                uint16_t h[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    h[e] = (k + e < p.k) ? __builtin_bit_cast(uint16_t, src[e]) : (uint16_t)0;
                }
                ra[i] = v4i{(int)(h[0] | (h[1] << 16)), (int)(h[2] | (h[3] << 16)),
                            (int)(h[4] | (h[5] << 16)), (int)(h[6] | (h[7] << 16))};
            }
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int idx = tid + i * T;
            const uint8_t* src;
            bool live;
            if constexpr (TRANS_B) {
                const int r = idx >> 1, kb = (k0 >> 5) + (idx & 1);
                live = kb < nbk;
                src = p.b + (int64_t)min(n0 + r, p.n - 1) * p.ldb + (int64_t)min(kb, nbk - 1) * 20;
            } else {
                const int kr = idx / (BN / 32), bn = (n0 >> 5) + idx % (BN / 32);
                live = (k0 + kr) < p.k;
                if constexpr (SOA) {
                    // the prepacked planes: d|m from its plane, nibble dword d
                    // of row r at 32 d + 4 (r % 8) of its group
                    const int64_t r = min(k0 + kr, p.k - 1);
                    const int64_t j = min(bn, nbn - 1);
                    const uint8_t* q = soa_group(p, j, r) + 4 * (r & 7);
                    rb[i][0] = live ? soa_dm(p, j, r) : 0u;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        rb[i][1 + d] = *reinterpret_cast<const uint32_t*>(q + 32 * d);
                    }
                    continue;
                }
                src = p.b + (int64_t)min(k0 + kr, p.k - 1) * p.ldb + (int64_t)min(bn, nbn - 1) * 20;
            }
            const v4i_a4 x = *reinterpret_cast<const v4i_a4*>(src);
            rb[i][0] = live ? (uint32_t)x.x : 0u;
            rb[i][1] = (uint32_t)x.y;
            rb[i][2] = (uint32_t)x.z;
            rb[i][3] = (uint32_t)x.w;
            rb[i][4] = *reinterpret_cast<const uint32_t*>(src + 16);
        }
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int idx = tid + i * T;
            const int r = idx >> 3, c = idx & 7;
            *reinterpret_cast<v4i*>(&lds_a[buf][r * kQLdsRow + c * 16]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int idx = tid + i * T;
            _Float16 w[32];
            decode_block_f16(rb[i], w);
            if constexpr (TRANS_B) {
                const int r = idx >> 1, kb = idx & 1;
                uint8_t* dst = &lds_b[buf][r * kQLdsRow + kb * 64];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    v4i v;
                    v.x = (int)(__builtin_bit_cast(uint16_t, w[8 * q + 0]) | (__builtin_bit_cast(uint16_t, w[8 * q + 1]) << 16));
                    v.y = (int)(__builtin_bit_cast(uint16_t, w[8 * q + 2]) | (__builtin_bit_cast(uint16_t, w[8 * q + 3]) << 16));
                    v.z = (int)(__builtin_bit_cast(uint16_t, w[8 * q + 4]) | (__builtin_bit_cast(uint16_t, w[8 * q + 5]) << 16));
                    v.w = (int)(__builtin_bit_cast(uint16_t, w[8 * q + 6]) | (__builtin_bit_cast(uint16_t, w[8 * q + 7]) << 16));
                    *reinterpret_cast<v4i*>(dst + q * 16) = v;
                }
            } else {
                const int kr = idx / (BN / 32), nb = idx % (BN / 32);
#pragma unroll
                for (int j = 0; j < 32; ++j) {
                    *reinterpret_cast<_Float16*>(&lds_b[buf][(nb * 32 + j) * kQLdsRow + kr * 2]) = w[j];
                }
            }
        }
    };

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            acc[i][j] = v16f{0.0f};
        }
    }

    const int kt = (p.k + kQBK - 1) / kQBK;
    load_stage(0);
    store_stage(0);
    __syncthreads();
    const int frow = lane & 31;
    const int fk = (lane >> 5) * 16;     // bytes: 8 halves per lane group
    for (int t = 0; t < kt; ++t) {
        const int cur = t & 1;
        if (t + 1 < kt) {
            load_stage((t + 1) * kQBK);
        }
#pragma unroll
        for (int ks = 0; ks < kQBK * 2; ks += 32) {    // 16 halves per MFMA step
            v8h fa[FM], fb[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                fa[i] = *reinterpret_cast<const v8h*>(&lds_a[cur][(wm0 + i * 32 + frow) * kQLdsRow + ks + fk]);
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                fb[j] = *reinterpret_cast<const v8h*>(&lds_b[cur][(wn0 + j * 32 + frow) * kQLdsRow + ks + fk]);
            }
#pragma unroll
            for (int i = 0; i < FM; ++i) {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (t + 1 < kt) {
            store_stage(cur ^ 1);
        }
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn0 + j * 32 + (lane & 31);
        if (n >= p.n) {
            continue;
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < p.m) {
                    store_out(p, m, n, acc[i][j][r]);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// MFMA GEMM for f32 A (nnops' f32 x q4_1 product is an f32 one): 128 x 128
// tiles, 4 waves of 64 x 64 (2 x 2 fragments of v_mfma_f32_32x32x2f32). Per
// 32-k stage (one block along K) A is staged as f32 rows and B decoded to f32
// (fmaf(d, q, m): d * q is exact, so one rounding, as d * q + m) as [n][k]
// rows, both with a 4-float pad. Lane group g (lane >> 5) owns k = 16 g ..
// 16 g + 15 of the stage for A and B alike (the MFMA's k index is the lane
// group, so any such assignment sums the same products), and a lane reads its
// 16 operands of a fragment with four 16-byte reads. FORM: 0 blocks along K
// ([N][K/32]); 1 blocks along N ([K][N/32] raw rows); 2 the prepacked planes
// of form 1. Bound: f32 MFMA.
// ---------------------------------------------------------------------------
template <int FORM>
__global__ __launch_bounds__(256, 1) void gemm_q4_1_f32(Q41Kern p)
{
    constexpr int BM = 128, BN = 128, LD = 36;
    __shared__ __attribute__((aligned(16))) float lds_a[2][BM * LD];
    __shared__ __attribute__((aligned(16))) float lds_b[2][BN * LD];

    const int tiles_n = (p.n + BN - 1) / BN;
    const int tm = blockIdx.x / tiles_n;
    const int tn = blockIdx.x - tm * tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave >> 1) * 64, wn0 = (wave & 1) * 64;
    const int nbn = (p.n + 31) / 32;
    const float* A = static_cast<const float*>(p.a);
    const bool a_vec = (p.lda & 3) == 0 && ((uintptr_t)A & 15) == 0;
    // B: thread -> block bi of the stage's 128, nibble bytes 8 bh .. 8 bh + 7
    // (values 8 bh .. 8 bh + 7 and 16 + 8 bh .. 16 + 8 bh + 7 of the block)
    const int bi = tid >> 1, bh = tid & 1;

    v4f ra[4];
    uint32_t rdm, rq0, rq1;
    auto load_stage = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = tid + i * 256;
            const int r = idx >> 3, c = idx & 7;      // 8 chunks of 4 floats per row
            const int k = k0 + 4 * c;
            const float* src = A + (int64_t)min(m0 + r, p.m - 1) * p.lda + k;
            if (a_vec && k + 4 <= p.k) {
                ra[i] = *reinterpret_cast<const v4f*>(src);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    ra[i][e] = k + e < p.k ? src[e] : 0.0f;
                }
            }
        }
        if constexpr (FORM == 0) {
            const uint8_t* src = p.b + (int64_t)min(n0 + bi, p.n - 1) * p.ldb + (int64_t)(k0 >> 5) * 20;
            rdm = *reinterpret_cast<const uint32_t*>(src);
            rq0 = *reinterpret_cast<const uint32_t*>(src + 4 + 8 * bh);
            rq1 = *reinterpret_cast<const uint32_t*>(src + 8 + 8 * bh);
        } else {
            const int kr = bi >> 2;
            const bool live = k0 + kr < p.k;
            const int64_t r = min(k0 + kr, p.k - 1);
            const int64_t j = min((n0 >> 5) + (bi & 3), nbn - 1);
            if constexpr (FORM == 1) {
                const uint8_t* src = p.b + r * p.ldb + j * 20;
                rdm = *reinterpret_cast<const uint32_t*>(src);
                rq0 = *reinterpret_cast<const uint32_t*>(src + 4 + 8 * bh);
                rq1 = *reinterpret_cast<const uint32_t*>(src + 8 + 8 * bh);
            } else {
                // nibble dword d of row r at 32 d + 4 (r % 8) of its group
                const uint8_t* q = soa_group(p, j, r) + 4 * (r & 7) + 64 * bh;
                rdm = soa_dm(p, j, r);
                rq0 = *reinterpret_cast<const uint32_t*>(q);
                rq1 = *reinterpret_cast<const uint32_t*>(q + 32);
            }
            rdm = live ? rdm : 0u;      // rows past K decode to 0
        }
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = tid + i * 256;
            *reinterpret_cast<v4f*>(&lds_a[buf][(idx >> 3) * LD + 4 * (idx & 7)]) = ra[i];
        }
        const float d = h2f(rdm & 0xffffu), mn = h2f(rdm >> 16);
        float lo[8], hi[8];
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint32_t byte = ((b < 4 ? rq0 : rq1) >> (8 * (b & 3))) & 0xffu;
            lo[b] = fmaf(d, (float)(byte & 15u), mn);
            hi[b] = fmaf(d, (float)(byte >> 4), mn);
        }
        if constexpr (FORM == 0) {
            float* row = &lds_b[buf][bi * LD];
            *reinterpret_cast<v4f*>(row + 8 * bh) = v4f{lo[0], lo[1], lo[2], lo[3]};
            *reinterpret_cast<v4f*>(row + 8 * bh + 4) = v4f{lo[4], lo[5], lo[6], lo[7]};
            *reinterpret_cast<v4f*>(row + 16 + 8 * bh) = v4f{hi[0], hi[1], hi[2], hi[3]};
            *reinterpret_cast<v4f*>(row + 16 + 8 * bh + 4) = v4f{hi[4], hi[5], hi[6], hi[7]};
        } else {
            const int kr = bi >> 2, c0 = (bi & 3) * 32 + 8 * bh;
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                lds_b[buf][(c0 + b) * LD + kr] = lo[b];
                lds_b[buf][(c0 + 16 + b) * LD + kr] = hi[b];
            }
        }
    };

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            acc[i][j] = v16f{0.0f};
        }
    }
    const int kt = (p.k + 31) / 32;
    const int fr = lane & 31, fg = 16 * (lane >> 5);
    load_stage(0);
    store_stage(0);
    __syncthreads();
    for (int t = 0; t < kt; ++t) {
        const int cur = t & 1;
        if (t + 1 < kt) {
            load_stage((t + 1) * 32);
        }
        v4f fa[2][4], fb[2][4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                fa[i][q] = *reinterpret_cast<const v4f*>(&lds_a[cur][(wm0 + 32 * i + fr) * LD + fg + 4 * q]);
                fb[i][q] = *reinterpret_cast<const v4f*>(&lds_b[cur][(wn0 + 32 * i + fr) * LD + fg + 4 * q]);
            }
        }
#pragma unroll
        for (int s = 0; s < 16; ++s) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][s >> 2][s & 3], fb[j][s >> 2][s & 3],
                                                                    acc[i][j], 0, 0, 0);
                }
            }
        }
        if (t + 1 < kt) {
            store_stage(cur ^ 1);
        }
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn0 + 32 * j + fr;
        if (n >= p.n) {
            continue;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm0 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < p.m) {
                    store_out(p, m, n, acc[i][j][r]);
                }
            }
        }
    }
}


// f32 A for the SPLIT ring: two f16 planes with a = (hi + lo) 2^e per row.
// The row's largest magnitude is scaled into [2^14, 2^15) (a power of two,
// exact), hi = RN_f16(a 2^-e) and lo = RN_f16(a 2^-e - hi) (the difference is
// exact in f32), so every value within 2^-28 of the row's largest keeps 22
// significant bits. One workgroup per row; e is clamped so 2^e and 2^-e are
// normal floats, and a row without a finite nonzero maximum keeps e = 0 (its
// infinities and NaNs pass into hi).
__global__ __launch_bounds__(256) void split_a_f32(const float* a, int64_t lda, int k, _Float16* hi, _Float16* lo,
                                                   float* row_scale)
{
    constexpr int kHold = 8;                 // 4-value groups a thread keeps between the passes (k <= 8192)
    __shared__ float red[4];
    const int m = blockIdx.x;
    const float* row = a + (int64_t)m * lda;
    // 16-byte loads where the row allows (k % 4 == 0 always: k % 64 == 0)
    const bool vec = ((uintptr_t)row & 15) == 0;
    auto load4 = [&](int i) {
        return vec ? *reinterpret_cast<const v4f*>(row + i) : v4f{row[i], row[i + 1], row[i + 2], row[i + 3]};
    };
    v4f held[kHold];
    float mx = 0.0f;
#pragma unroll
    for (int u = 0; u < kHold; ++u) {
        const int i = 4 * (int)threadIdx.x + 1024 * u;
        held[u] = i < k ? load4(i) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int u = 0; u < kHold; ++u) {
        mx = fmaxf(fmaxf(mx, __builtin_fabsf(held[u][0])), __builtin_fabsf(held[u][1]));
        mx = fmaxf(fmaxf(mx, __builtin_fabsf(held[u][2])), __builtin_fabsf(held[u][3]));
    }
    for (int i = 4 * (int)threadIdx.x + 1024 * kHold; i < k; i += 1024) {
        const v4f x = load4(i);
        mx = fmaxf(fmaxf(mx, __builtin_fabsf(x[0])), __builtin_fabsf(x[1]));
        mx = fmaxf(fmaxf(mx, __builtin_fabsf(x[2])), __builtin_fabsf(x[3]));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    }
    if ((threadIdx.x & 63) == 0) {
        red[threadIdx.x >> 6] = mx;
    }
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (mx > 0.0f && mx <= 3.402823466e38f) {
        // the exponent of mx (a subnormal one counts as -127: clamped below)
        const int ex = (int)((__float_as_uint(mx) >> 23) & 0xffu) - 127;
        e = min(max(ex - 14, -126), 113);
    }
    const float down = __uint_as_float((uint32_t)(127 - e) << 23);    // 2^-e
    if (threadIdx.x == 0) {
        row_scale[m] = __uint_as_float((uint32_t)(127 + e) << 23);    // 2^e
    }
    _Float16* h_row = hi + (int64_t)m * k;
    _Float16* l_row = lo + (int64_t)m * k;
    auto put4 = [&](int i, const v4f& x) {
        _Float16 h[4], l[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float y = x[q] * down;
            h[q] = (_Float16)y;
            l[q] = (_Float16)(y - (float)h[q]);
        }
        uint2 hw, lw;
        __builtin_memcpy(&hw, h, 8);
        __builtin_memcpy(&lw, l, 8);
        *reinterpret_cast<uint2*>(h_row + i) = hw;
        *reinterpret_cast<uint2*>(l_row + i) = lw;
    };
#pragma unroll
    for (int u = 0; u < kHold; ++u) {
        const int i = 4 * (int)threadIdx.x + 1024 * u;
        if (i < k) {
            put4(i, held[u]);
        }
    }
    for (int i = 4 * (int)threadIdx.x + 1024 * kHold; i < k; i += 1024) {
        put4(i, load4(i));
    }
}

// ---------------------------------------------------------------------------
// MFMA GEMM, f16 A, B blocks along K ([N][K/32], 2 blocks = 40 bytes per row
// per 64-k stage), K % 64 == 0. 128 x 256 tiles, WM x WN waves (the launch
// uses 1 x 8: each wave 128 x 32, two per SIMD) of 32x32 fragments
// (v_mfma_f32_32x32x16_f16), an NS-stage LDS ring filled only by
// buffer_load ... lds (so every wait below is an explicit vmcnt):
//   A     128 rows x 128 bytes; 16-byte chunk c of row r in slot c ^ ((r >> 1) & 7)
//   Braw  256 rows x 64 bytes (the row's 40 stage bytes + 24 not used); chunk
//         c of row r in slot c ^ ((r >> 2) & 3)
// Both swizzles make the 16- and 4-byte fragment reads of 32 consecutive rows
// conflict-free (A) or at most 2-way (Braw). Each lane decodes its own B
// operand in registers: 8 nibbles of one row (a dword pair) and the block's
// d | m dword become 8 f16 d * q + m: the byte permute with exponent byte 0x64
// makes (1024 + q, 1024 + q'), v_pk_add_f16 removes 1024 exactly and
// v_pk_fma_f16 rounds d * q + m once. Stage s + NS - 1 is issued at the top of
// step s and has NS - 2 steps to land. Bound: MFMA.
// ---------------------------------------------------------------------------
// 8 nibble values (low nibble of each byte of lo0, lo1) -> 8 f16 d * q + m
__device__ __forceinline__ v8h decode8_f16(uint32_t lo0, uint32_t lo1, v2h d2, v2h m2)
{
    const v2h k1024 = __builtin_bit_cast(v2h, 0x64006400u);
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t src = i ? lo1 : lo0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t pr = __builtin_amdgcn_perm(0x64646464u, src, h ? 0x04030402u : 0x04010400u);
            const v2h q = __builtin_bit_cast(v2h, pr) - k1024;
            w[2 * i + h] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, d2, m2));
        }
    }
    return __builtin_bit_cast(v8h, v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]});
}

// GATED: Linear's gated form with its output pass p.fo fused: the tile covers
// output columns 128 tn .. + 127 and stages the weight's gate rows there and
// its value rows (N / 2 further) in its second half, so waves 0-3 hold the
// gate products and waves 4-7 the value products of the same columns, which
// meet through LDS for the combine. (Fusing the plain pass -- bias, residual,
// activation -- measured slower than the separate pass: 108 against 98 us at
// 512 x 14336 x 4096, the pass's arithmetic then running with the matrix
// cores idle; the gated form saves the larger staging: 196 -> 184 us.)
template <bool OUT16, int NS, int WM, int WN = 4, bool GATED = false, bool SPLIT = false, int BM = 128, int BN = 256>
__global__ __launch_bounds__(64 * WM * WN, 1) void gemm_q4_1_ring(Q41Kern p)
{
    static_assert(!GATED || (WM == 1 && WN == 8 && BM == 128 && BN == 256),
                  "gated: one wave per 32 columns, halves 4 waves apart");
    static_assert(!SPLIT || (!GATED && WM == 1), "split A: one wave row");
    constexpr int W = WM * WN;                      // waves: WM along M x WN along N
    constexpr int AP = SPLIT ? 2 : 1;               // planes of A (SPLIT: hi and lo f16 parts)
    constexpr int QA = AP * BM / (8 * W), QB = BN / (16 * W);   // 1 KiB pieces per wave per stage
    static_assert(QA * 8 * W == AP * BM && QB * 16 * W == BN, "whole pieces per wave");
    constexpr int L = QA + QB;
    static_assert(NS >= 3 && (NS - 2) * L < 64, "stages");
    constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    constexpr int kA = AP * BM * 128, kB = BN * 64, kStage = kA + kB;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[NS * kStage];

    const int tiles_m = (p.m + BM - 1) / BM;
    int bid = blockIdx.x;
    const int nb = gridDim.x;
    if ((nb & 7) == 0) {
        bid = (bid & 7) * (nb >> 3) + (bid >> 3);     // consecutive logical tiles on one XCD
    }
    const int tm = bid % tiles_m, tn = bid / tiles_m; // the M tiles of a column band share B in L2
    const int m0 = tm * BM;
    const int n0 = GATED ? tn * (BN / 2) : tn * BN;   // gated: output columns; the weight has 2 p.fo.n rows
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wn0 = (wave % WN) * TN;
    const int wm0 = (wave / WN) * TM;
    const int kt = p.k / 64;

    // A: rows 8 * (4 * wave + i) + lane / 8; B raw: rows 16 * (4 * wave + i) + lane / 4
    const QBufRsrc rsa = q_buffer_rsrc(static_cast<const _Float16*>(p.a) + (int64_t)m0 * p.lda, 0x7fffffffu);
    const int64_t b_bytes = (int64_t)(p.n - (GATED ? 0 : n0)) * p.ldb;
    const QBufRsrc rsb = q_buffer_rsrc(p.b + (GATED ? 0 : (int64_t)n0 * p.ldb),
                                       (uint32_t)std::min<int64_t>(b_bytes, 0x7fffffff));
    int a_off[QA], b_off[QB];
#pragma unroll
    for (int i = 0; i < QA; ++i) {
        // SPLIT: staged rows 128..255 are the lo plane's rows 0..127
        const int ra = 8 * (QA * wave + i) + (lane >> 3);
        const int ca = (lane & 7) ^ ((ra >> 1) & 7);
        a_off[i] = min(ra & (BM - 1), p.m - 1 - m0) * (int)p.lda * 2 + ca * 16 + (ra >= BM ? (int)p.plane : 0);
    }
#pragma unroll
    for (int i = 0; i < QB; ++i) {
        const int rb = 16 * (QB * wave + i) + (lane >> 2);
        const int cb = (lane & 3) ^ ((rb >> 2) & 3);
        if constexpr (GATED) {
            // tile rows 0..127: gate rows n0 + rb; 128..255: value rows
            // p.fo.n + n0 + rb - 128 (each half clamped to its own rows)
            const int half = rb >> 7, r = min(n0 + (rb & 127), p.fo.n - 1);
            b_off[i] = (half * p.fo.n + r) * (int)p.ldb + cb * 16;
        } else {
            b_off[i] = min(rb, p.n - 1 - n0) * (int)p.ldb + cb * 16;
        }
    }
    auto issue = [&](int s) {
        uint8_t* base = ring + (s % NS) * kStage;
#pragma unroll
        for (int i = 0; i < QA; ++i) {
            q_buffer_load_lds16(rsa, base + (QA * wave + i) * 1024, a_off[i], s * 128);
        }
#pragma unroll
        for (int i = 0; i < QB; ++i) {
            q_buffer_load_lds16(rsb, base + kA + (QB * wave + i) * 1024, b_off[i], s * 40);
        }
    };

    // this lane's fragment rows: A row (lane & 31) of fragment i; B row
    // wn0 + 32 j + (lane & 31); k values 16 ks + 8 (lane >> 5) .. + 7
    const int fr = lane & 31, kh = lane >> 5;
    auto a_frag = [&](const uint8_t* st, int i, int ks) {
        const int r = (i >= FM ? BM : 0) + wm0 + (i % FM) * 32 + fr;
        const int c = (2 * ks + kh) ^ ((r >> 1) & 7);
        return *reinterpret_cast<const v8h*>(st + r * 128 + c * 16);
    };
    auto b_dword = [&](const uint8_t* row, int r, int byte) {
        const int c = (byte >> 4) ^ ((r >> 2) & 3);
        return *reinterpret_cast<const uint32_t*>(row + c * 16 + (byte & 15));
    };
    // B fragments of both slices of one block (ks = 2 blk, 2 blk + 1): the
    // lane's 8 nibble bytes hold its values of the first slice in their low
    // nibbles and of the second in their high ones, so one read of d/m and
    // the 8 bytes decodes both
    auto b_frag2 = [&](const uint8_t* st, int j, int blk, v8h& lo, v8h& hi) {
        const int r = wn0 + 32 * j + fr;
        const uint8_t* row = st + kA + r * 64;
        const uint32_t dm = b_dword(row, r, 20 * blk);
        const int nb0 = 20 * blk + 4 + 8 * kh;               // first nibble byte
        const uint32_t w0 = b_dword(row, r, nb0), w1 = b_dword(row, r, nb0 + 4);
        const v2h d2 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(dm, dm, 0x01000100u));
        const v2h m2 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(dm, dm, 0x03020302u));
        lo = decode8_f16(w0 & 0x0f0f0f0fu, w1 & 0x0f0f0f0fu, d2, m2);
        hi = decode8_f16((w0 >> 4) & 0x0f0f0f0fu, (w1 >> 4) & 0x0f0f0f0fu, d2, m2);
    };

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            acc[i][j] = v16f{0.0f};
        }
    }

    // prologue: stages 0..NS-2 in flight, stage 0 landed
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) {
        if (s < kt) {
            issue(s);
        }
    }
    if (kt >= NS - 1) {
        wait_vmcnt<(NS - 2) * L>();
    } else {
        wait_vmcnt<0>();
    }
    __syncthreads();

    // Within a step the fragments of the next slice are read and decoded
    // while the matrix cores run this one (B for both slices of a block at
    // once; two register sets, alternating).
    v8h fa0[AP * FM], fb0[FN], fa1[AP * FM], fb1[FN], fb2[FN], fb3[FN];
    auto load_a = [&](const uint8_t* st, int ks, v8h (&fa)[AP * FM]) {
#pragma unroll
        for (int i = 0; i < AP * FM; ++i) {
            fa[i] = a_frag(st, i, ks);
        }
    };
    auto load_b = [&](const uint8_t* st, int blk, v8h (&lo)[FN], v8h (&hi)[FN]) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            b_frag2(st, j, blk, lo[j], hi[j]);
        }
    };
    // SPLIT: the hi parts' products first, then the lo parts' into the same
    // accumulators (FM * FN independent products apart)
    auto mfma_slice = [&](const v8h (&fa)[AP * FM], const v8h (&fb)[FN]) {
#pragma unroll
        for (int h = 0; h < AP; ++h) {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
#pragma unroll
                for (int i = 0; i < FM; ++i) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[h * FM + i], fb[j], acc[i][j], 0, 0, 0);
                }
            }
        }
    };
    for (int t = 0; t < kt; ++t) {
        const uint8_t* st = ring + (t % NS) * kStage;
        // stage t+NS-1 into the slot read in step t-1
        const bool more = t + NS - 1 < kt;
        if (more) {
            issue(t + NS - 1);
        }
        load_b(st, 0, fb0, fb1);
        load_a(st, 0, fa0);
        load_a(st, 1, fa1);
        mfma_slice(fa0, fb0);
        load_b(st, 1, fb2, fb3);
        load_a(st, 2, fa0);
        mfma_slice(fa1, fb1);
        load_a(st, 3, fa1);
        mfma_slice(fa0, fb2);
        mfma_slice(fa1, fb3);
        // stage t+1 landed for this wave (issued NS-2 steps ago; every later
        // stage may be in flight); the barrier makes every wave's pieces visible
        // and frees slot t for step t+1's issue
        if (more) {
            wait_vmcnt<(NS - 2) * L>();
        } else {
            wait_vmcnt<0>();
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    }

    // C[m][n]: lane holds column n = (lane & 31) of fragment j, rows 8 (r / 4) + 4 (lane >> 5) + r % 4
    // The gated combine. The pass is too large to inline once per register
    // (a call would put its parameters on the stack), so the products go
    // through the ring (free once every wave is past it) and a loop of a few
    // rows per step applies it: xs[wave][i * 16 + r][lane] is product row
    // 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4 of the wave's column lane % 32.
    // Gate wave w (0-3) and value wave w + 4 hold the two products of the
    // same outputs; the gate wave combines rows 0-63, the value wave 64-127.
    if constexpr (GATED) {
        static_assert(W * FM * 16 * 64 * 4 <= NS * kStage, "the products fit the ring");
        const FpOut fo = p.fo;
        __syncthreads();
        float* xs = reinterpret_cast<float*>(ring);
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                xs[((wave * FM + i) * 16 + r) * 64 + lane] = acc[i][0][r];
            }
        }
        __syncthreads();
        const int gw = wave & 3;
        const int n = n0 + gw * 32 + (lane & 31);
        if (n >= fo.n) {
            return;
        }
        const float bg = bias_at(fo, n), bu = bias_at(fo, fo.n + n);
        const int first = wave >= 4 ? FM * 8 : 0;
#pragma unroll 4
        for (int q = 0; q < FM * 8; ++q) {
            const int ir = first + q, i = ir >> 4, r = ir & 15;
            const int m = m0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m < p.m) {
                char* orow = static_cast<char*>(fo.out) + (int64_t)m * fo.ld_out * (fo.out_f16 ? 2 : 4);
                const float g = xs[((gw * FM) * 16 + ir) * 64 + lane];
                const float v = xs[(((gw + 4) * FM) * 16 + ir) * 64 + lane];
                fp_out_store(fo, orow, n, fp_out_value(fo, g, v, fp_out_old(fo, orow, n), bg, bu));
            }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn0 + j * 32 + (lane & 31);
        if (n >= p.n) {
            continue;
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < p.m) {
                    // SPLIT: the row's power-of-two factor (exact)
                    const float v = SPLIT ? acc[i][j][r] * p.row_scale[m] : acc[i][j][r];
                    if constexpr (OUT16) {
                        __builtin_nontemporal_store((_Float16)v, static_cast<_Float16*>(p.c) + (int64_t)m * p.ldc + n);
                    } else {
                        __builtin_nontemporal_store(v, static_cast<float*>(p.c) + (int64_t)m * p.ldc + n);
                    }
                }
            }
        }
    }
}


// ---------------------------------------------------------------------------
// MFMA GEMM, f16 A, B blocks along N ([K][N/32]: each k row holds one 20-byte
// block per 32 columns), K % 64 == 0. Same 128 x 256 tile, 8 waves of 128 x
// 32 (wave w owns the tile's block column w) and NS-stage DMA ring as
// gemm_q4_1_ring; only B's staging and decode differ:
//   Braw  the stage's 64 k rows x 160 bytes (the tile's 8 blocks of each row,
//         contiguous in memory), 640 16-byte chunks; row k sits at slot row
//         k ^ ((k >> 3) & 1), so the two lane halves of a fragment (rows k and
//         k + 8) land 24 or 40 banks apart.
// A lane's B operand is column n = lane & 31 of its wave's block at 8
// consecutive k rows: per row the block's d | m dword (one address per lane
// half: a broadcast read) and the nibble dword holding byte n & 15, nibble
// n >> 4. Two rows decode per step: the byte permute pulls the lane's byte of
// both rows, shift and mask keep the nibble under exponent byte 0x64, and
// v_pk_fma_f16 applies the two rows' own d and m.
// SOA: B is the prepacked form (nibble plane + d|m plane): a stage holds the
// tile's 64 x 128 nibble bytes (8 pieces, one per wave) and then its 64 x 32
// d|m bytes (2 pieces, waves 0 and 1), both with the slot-row order above
// (rows k and k + 8 then sit 32 banks apart in the nibbles and 8 in d|m).
// ---------------------------------------------------------------------------
template <bool OUT16, int NS, bool SOA, bool SPLIT = false>
__global__ __launch_bounds__(512, 1) void gemm_q4_1_kn_ring(Q41Kern p)
{
    constexpr int AP = SPLIT ? 2 : 1;               // planes of A (SPLIT: hi and lo f16 parts)
    constexpr int W = 8, QA = 2 * AP;               // A: 2 KiB pieces per wave per stage and plane
    constexpr int BM = 128, BN = 256, FM = 4;
    constexpr int kRow = BN / 32 * 20;              // 160 bytes of B per k row
    // slot-row pitch of the d|m dwords and of the nibble dwords, and where the
    // d|m rows start within the stage's B
    constexpr int kRowD = SOA ? BN / 32 * 4 : kRow, kRowQ = SOA ? BN / 32 * 16 : kRow;
    // SOA nibbles: one 1 KiB piece per group of 8 rows (the tile's 8 blocks x
    // 128 bytes), pieces 1040 bytes apart so that the two lane halves' groups
    // (2 ks and 2 ks + 1) sit 4 banks apart; the d|m rows follow
    constexpr int kGrp = 1040;
    constexpr int kDmAt = SOA ? 8 * kGrp : 0;
    constexpr int kA = AP * BM * 128, kB = SOA ? kDmAt + 64 * kRowD : 64 * kRow, kStage = kA + kB;
    constexpr int kBPieces = kB / 1024;             // 10 x 1 KiB: waves 0, 1 issue two
    static_assert(NS >= 3 && kBPieces > W && kBPieces <= 2 * W, "stages");
    __shared__ __attribute__((aligned(1024))) uint8_t ring[NS * kStage];

    const int tiles_m = (p.m + BM - 1) / BM;
    int bid = blockIdx.x;
    const int nb = gridDim.x;
    if ((nb & 7) == 0) {
        bid = (bid & 7) * (nb >> 3) + (bid >> 3);     // consecutive logical tiles on one XCD
    }
    const int tm = bid % tiles_m, tn = bid / tiles_m; // the M tiles of a column band share B in L2
    const int m0 = tm * BM, n0 = tn * BN;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kt = p.k / 64;
    const bool two = wave < kBPieces - W;

    const QBufRsrc rsa = q_buffer_rsrc(static_cast<const _Float16*>(p.a) + (int64_t)m0 * p.lda, 0x7fffffffu);
    // this tile's blocks of row 0; a stage's rows start s * 64 * ldb further
    const int nbn = (p.n + 31) / 32;
    // SOA: the tile's first block column of each plane; a stage is 8 groups
    // (1 KiB) further along every block column's nibbles, 256 bytes along its
    // d|m dwords
    const uint8_t* b0 = p.b + (int64_t)(n0 / 32) * (SOA ? p.ldb : 20);
    const int64_t b_end = SOA ? (int64_t)(nbn - n0 / 32) * p.ldb
                              : (int64_t)(p.k - 1) * p.ldb + (int64_t)(nbn - n0 / 32) * 20;
    const int64_t ldd = p.ldbdm * 4;                // SOA: d|m block column pitch in bytes
    const uint8_t* d0 = reinterpret_cast<const uint8_t*>(p.bdm) + (int64_t)(n0 / 32) * ldd;
    const int64_t d_end = (int64_t)(nbn - n0 / 32) * ldd;
    const int last_blk = nbn - 1 - n0 / 32;         // blocks past N re-read the last one
    int a_off[QA], b_off[2];
#pragma unroll
    for (int i = 0; i < QA; ++i) {
        // SPLIT: staged rows 128..255 are the lo plane's rows 0..127
        const int ra = 8 * (QA * wave + i) + (lane >> 3);
        const int ca = (lane & 7) ^ ((ra >> 1) & 7);
        a_off[i] = min(ra & (BM - 1), p.m - 1 - m0) * (int)p.lda * 2 + ca * 16 + (ra >= BM ? (int)p.plane : 0);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int q = (wave + W * i) * 64 + lane;     // chunk = LDS slot
        if constexpr (SOA) {
            // nibble piece: the wave's group of 8 rows, 128 bytes from each
            // of the tile's 8 block columns; d|m pieces: 16 chunks of 4 rows
            // per block column, [block][row] in the slot
            if (i == 0) {
                b_off[i] = min(lane >> 3, last_blk) * (int)p.ldb + wave * 128 + (lane & 7) * 16;
            } else {
                const int qq = q - W * 64;
                b_off[i] = min(qq >> 4, last_blk) * (int)ldd + (qq & 15) * 16;
            }
        } else {
            const int pr = q / 10, c = q - pr * 10;
            const int k = pr ^ ((pr >> 3) & 1);
            b_off[i] = k * (int)p.ldb + c * 16;
        }
    }
    auto issue = [&](int s) {
        uint8_t* base = ring + (s % NS) * kStage;
#pragma unroll
        for (int i = 0; i < QA; ++i) {
            q_buffer_load_lds16(rsa, base + (QA * wave + i) * 1024, a_off[i], s * 128);
        }
        const int64_t row0 = SOA ? (int64_t)s * 1024 : (int64_t)s * 64 * p.ldb;
        const QBufRsrc rsb = q_buffer_rsrc(b0 + row0, (uint32_t)std::min<int64_t>(b_end - row0, 0x7fffffff));
        q_buffer_load_lds16(rsb, base + kA + wave * (SOA ? kGrp : 1024), b_off[0], 0);
        if (two) {
            if constexpr (SOA) {
                const int64_t drow0 = (int64_t)s * 256;
                const QBufRsrc rsd =
                    q_buffer_rsrc(d0 + drow0, (uint32_t)std::min<int64_t>(d_end - drow0, 0x7fffffff));
                q_buffer_load_lds16(rsd, base + kA + kDmAt + wave * 1024, b_off[1], 0);
            } else {
                q_buffer_load_lds16(rsb, base + kA + (wave + W) * 1024, b_off[1], 0);
            }
        }
    };
    auto wait_ring = [&](bool full) {
        if (full) {
            wait_vmcnt<0>();
        } else if (two) {
            wait_vmcnt<(NS - 2) * (QA + 2)>();
        } else {
            wait_vmcnt<(NS - 2) * (QA + 1)>();
        }
    };

    const int fr = lane & 31, kh = lane >> 5;
    auto a_frag = [&](const uint8_t* st, int i, int ks) {
        const int r = (i >= FM ? BM : 0) + (i % FM) * 32 + fr;
        const int c = (2 * ks + kh) ^ ((r >> 1) & 7);
        return *reinterpret_cast<const v8h*>(st + r * 128 + c * 16);
    };
    // per-lane constants of the B decode: the block's byte offset in a row,
    // the nibble dword, and the permute picking byte n & 3 of two rows into
    // bytes 0 and 2
    const int bcol = SOA ? kDmAt + 4 * wave : 20 * wave;
    const int qdw = SOA ? 16 * wave + 4 * ((fr & 15) >> 2) : bcol + 4 + 4 * ((fr & 15) >> 2);
    const uint32_t qsel = 0x0c000c00u | ((uint32_t)(4 + (fr & 3)) << 16) | (uint32_t)(fr & 3);
    // Rows 16 ks + 8 kh + e, e + 1 (e even) sit at slot rows 16 ks + e + 9 kh
    // and 16 ks + e + 1 + 7 kh: a lane base per row of the pair, the rest are
    // immediate offsets
    const int sr0 = 9 * kh, sr1 = 7 * kh + 1;
    const int bxs = kA + kh * kGrp + 128 * wave + 32 * ((fr & 15) >> 2);   // SOA nibbles
    const int bds = kA + kDmAt + 256 * wave + 32 * kh;                     // SOA d|m: rows 8 kh ..
    const int bd0 = kA + sr0 * kRowD + bcol, bq0 = kA + sr0 * kRowQ + qdw;
    const int bd1 = kA + sr1 * kRowD + bcol, bq1 = kA + sr1 * kRowQ + qdw;
    // Low-nibble lanes keep 0x0f under exponent byte 0x64: f16 1024 + q.
    // High-nibble lanes keep 0xf0 under 0x54: in [64, 128) a mantissa unit is
    // 1/16, so the nibble's bits 4-7 read as 64 + q. Each subtracts its own
    // bias, exactly, and no lane shifts.
    const bool hi_nib = fr >= 16;
    const uint32_t kMask = hi_nib ? 0x00f000f0u : 0x000f000fu;
    const uint32_t kMagic = hi_nib ? 0x54005400u : 0x64006400u;
    const v2h kBias = __builtin_bit_cast(v2h, kMagic);
    // B fragment of slice ks in two steps, so that the next slice's reads are
    // in flight while this one decodes: 16 raw dwords, then 8 f16 values
    struct BRaw {
        uint32_t dm0[4], dm1[4], x0[4], x1[4];
    };
    auto b_read = [&](const uint8_t* st, int ks, BRaw& r) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int od = (16 * ks + 2 * e) * kRowD, oq = (16 * ks + 2 * e) * kRowQ;
            if constexpr (SOA) {
                // rows 16 ks + 8 kh + 2 e and + 1 of the wave's block column
                const v2u32 dd = *reinterpret_cast<const v2u32*>(st + bds + (16 * ks + 2 * e) * 4);
                r.dm0[e] = dd.x;
                r.dm1[e] = dd.y;
            } else {
                r.dm0[e] = *reinterpret_cast<const uint32_t*>(st + bd0 + od);
                r.dm1[e] = *reinterpret_cast<const uint32_t*>(st + bd1 + od);
                r.x0[e] = *reinterpret_cast<const uint32_t*>(st + bq0 + oq);
                r.x1[e] = *reinterpret_cast<const uint32_t*>(st + bq1 + oq);
            }
        }
        if constexpr (SOA) {
            // the lane's dword of its block for the 8 rows of group 2 ks + kh
            const v4i* xs = reinterpret_cast<const v4i*>(st + bxs + 2 * ks * kGrp);
            const v4i lo = xs[0], hi = xs[1];
            r.x0[0] = (uint32_t)lo.x, r.x1[0] = (uint32_t)lo.y, r.x0[1] = (uint32_t)lo.z, r.x1[1] = (uint32_t)lo.w;
            r.x0[2] = (uint32_t)hi.x, r.x1[2] = (uint32_t)hi.y, r.x0[3] = (uint32_t)hi.z, r.x1[3] = (uint32_t)hi.w;
        }
    };
    auto b_decode = [&](const BRaw& r) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint32_t t;
            asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(t) : "v"(__builtin_amdgcn_perm(r.x1[e], r.x0[e], qsel)),
                "v"(kMask), "v"(kMagic));
            const v2h q = __builtin_bit_cast(v2h, t) - kBias;
            const v2h d2 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(r.dm1[e], r.dm0[e], 0x05040100u));
            const v2h m2 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(r.dm1[e], r.dm0[e], 0x07060302u));
            w[e] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, d2, m2));
        }
        return __builtin_bit_cast(v8h, v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]});
    };

    v16f acc[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        acc[i] = v16f{0.0f};
    }

#pragma unroll
    for (int s = 0; s < NS - 1; ++s) {
        if (s < kt) {
            issue(s);
        }
    }
    wait_ring(kt < NS - 1);
    __syncthreads();

    v8h fa0[AP * FM], fa1[AP * FM], fb0, fb1;
    auto load_a = [&](const uint8_t* st, int ks, v8h (&fa)[AP * FM]) {
#pragma unroll
        for (int i = 0; i < AP * FM; ++i) {
            fa[i] = a_frag(st, i, ks);
        }
    };
    // SPLIT: the hi parts' products, then the lo parts' into the same accumulators
    auto mfma_slice = [&](const v8h (&fa)[AP * FM], const v8h& fb) {
#pragma unroll
        for (int h = 0; h < AP; ++h) {
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[h * FM + i], fb, acc[i], 0, 0, 0);
            }
        }
    };
    for (int t = 0; t < kt; ++t) {
        const uint8_t* st = ring + (t % NS) * kStage;
        const bool more = t + NS - 1 < kt;
        if (more) {
            issue(t + NS - 1);
        }
        BRaw r0, r1;
        b_read(st, 0, r0);
        load_a(st, 0, fa0);
        b_read(st, 1, r1);
        fb0 = b_decode(r0);
        load_a(st, 1, fa1);
        b_read(st, 2, r0);
        mfma_slice(fa0, fb0);
        fb1 = b_decode(r1);
        load_a(st, 2, fa0);
        b_read(st, 3, r1);
        mfma_slice(fa1, fb1);
        fb0 = b_decode(r0);
        load_a(st, 3, fa1);
        mfma_slice(fa0, fb0);
        fb1 = b_decode(r1);
        mfma_slice(fa1, fb1);
        wait_ring(!more);
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    }

    const int n = n0 + 32 * wave + fr;
    if (n < p.n) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + i * 32 + 8 * (r >> 2) + 4 * kh + (r & 3);
                if (m < p.m) {
                    // SPLIT: the row's power-of-two factor (exact)
                    const float v = SPLIT ? acc[i][r] * p.row_scale[m] : acc[i][r];
                    if constexpr (OUT16) {
                        __builtin_nontemporal_store((_Float16)v, static_cast<_Float16*>(p.c) + (int64_t)m * p.ldc + n);
                    } else {
                        __builtin_nontemporal_store(v, static_cast<float*>(p.c) + (int64_t)m * p.ldc + n);
                    }
                }
            }
        }
    }
}


// ---------------------------------------------------------------------------
// Prepack of a blocks-along-N weight into its two planes (structure of
// arrays), one block column after another: thread per block; the nibble
// plane is k-blocked (block column j: per 8 rows, per nibble dword, the 8
// rows' dwords, 32 bytes), the d|m dword goes to row r of block column j of
// its plane; padding (rows past K) is zeroed.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prepack_q4_1_kn(const uint8_t* b, int64_t ldb, int k, int nbn,
                                                       uint8_t* nib, uint32_t* dm, int64_t kdm)
{
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)k * nbn) {
        return;
    }
    const int64_t r = idx / nbn;
    const int j = (int)(idx - r * nbn);
    const uint32_t* src = reinterpret_cast<const uint32_t*>(b + r * ldb + (int64_t)j * 20);
    const int64_t kg = (k + 7) / 8;
    uint32_t* g = reinterpret_cast<uint32_t*>(nib + ((int64_t)j * kg + (r >> 3)) * 128);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        g[8 * d + (r & 7)] = src[1 + d];
    }
    dm[(int64_t)j * kdm + r] = src[0];
    if (r == k - 1) {
        // the last group's rows past K, and the block column's d|m rows past K
        for (int rr = (int)(r & 7) + 1; rr < 8; ++rr) {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                g[8 * d + rr] = 0u;
            }
        }
        for (int64_t t = k; t < kdm; ++t) {
            dm[(int64_t)j * kdm + t] = 0u;
        }
    }
}

constexpr size_t kAlign = 256;

inline size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

inline int kn_splits(const NnopsGemmQ41Args& g)
{
    // about 1024 workgroups (16 blocks wide each), at least 64 k rows per split
    const int64_t ncol = ((g.n + 31) / 32 + 15) / 16;
    int64_t s = (1024 + ncol - 1) / ncol;
    s = std::min<int64_t>(s, std::max<int64_t>(1, g.k / 64));
    return (int)std::max<int64_t>(1, std::min<int64_t>(s, 256));
}

// The one-launch blocks-along-N GEMV (gemv_q4_1_kn_dma): raw rows (not the
// prepacked planes), f16 A with 4-byte-aligned row pairs (even K), 16-byte rows, and
// each split's row range within a 31-bit buffer offset.
struct KnDmaPlan {
    int groups = 0, splits = 0, kper = 0;
};

inline KnDmaPlan plan_kn_dma(const NnopsGemmQ41Args& g)
{
    KnDmaPlan r;
    if (g.trans_b || g.b_soa || !g.a_f16 || (g.ldb_bytes % 16) != 0 || ((uintptr_t)g.b & 15) != 0 ||
        ((uintptr_t)g.a & 3) != 0 || (g.lda % 2) != 0 || (g.k % 2) != 0) {
        return r;
    }
    const int64_t groups = ((g.n + 31) / 32 + 31) / 32;
    // about two workgroups per CU, whole 32-row stages
    const int64_t want = std::max<int64_t>(1, (512 + groups - 1) / groups);
    int64_t kper = ((g.k + want - 1) / want + 31) / 32 * 32;
    kper = std::max<int64_t>(kper, 32);
    if ((kper + 32) * g.ldb_bytes >= (int64_t)INT32_MAX || groups > 65535) {
        return r;
    }
    r.groups = (int)groups;
    r.kper = (int)kper;
    r.splits = (int)((g.k + kper - 1) / kper);
    if (r.splits > 64) {             // one flag per lane of a wave
        r.kper = (int)(((g.k + 63) / 64 + 31) / 32 * 32);
        r.splits = (int)((g.k + r.kper - 1) / r.kper);
        if ((int64_t)(r.kper + 32) * g.ldb_bytes >= (int64_t)INT32_MAX) {
            return KnDmaPlan{};
        }
    }
    return r;
}

inline size_t kn_dma_part_bytes(const KnDmaPlan& r)
{
    return (size_t)r.groups * r.splits * 2 * 4096;
}

// f32 A: the GEMV loop (one row of A per pass, each pass streaming the whole
// weight) up to this many rows, the f32 MFMA GEMM past them. At K = 4096,
// N = 14336 a pass takes 17-18 us and the GEMM 300 us for any M <= 128 (one
// 128 x 128 tile per workgroup, 112 of them), 550 us at M = 512.
constexpr int64_t kF32GemvRows = 16;

inline bool use_gemv(const NnopsGemmQ41Args& g)
{
    return g.m <= 2 || (!g.a_f16 && g.m <= kF32GemvRows);
}

// The blocks-along-N ring: f16 A with 16-byte rows, K % 64 == 0, 16-byte B
// rows, and every stage offset within a buffer resource's 31-bit range
// The skinny MFMA GEMM (gemv_q4_1_skinny): blocks along K, f16 A with 16-byte
// rows, 3 <= M <= 48 (launches of 16 rows), K % 256 == 0, 16-byte weight rows,
// 32-bit offsets. At K = 4096, N = 14336 a launch takes 16 us, the ring 58-62
// us for any M <= 128: past three launches the ring is the faster.
constexpr int64_t kSkinnyMaxM = 48;

inline bool skinny_ok(const NnopsGemmQ41Args& g)
{
    const int64_t es = g.a_f16 ? 2 : 4;
    return g.trans_b && !g.b_soa && g.m >= 3 && g.m <= kSkinnyMaxM && g.k % 256 == 0 &&
           (g.ldb_bytes % 16) == 0 && ((uintptr_t)g.b & 15) == 0 && (g.lda * es) % 16 == 0 &&
           ((uintptr_t)g.a & 15) == 0 && 32 * g.ldb_bytes < INT32_MAX && g.m * g.lda * es < INT32_MAX;
}

// rows of A up to which the prepacked planes take the GEMV passes rather than
// the ring (M = 12: 65 us against 77), and (K % 256 == 0) the skinny MFMA
// form, one launch per 16 rows
constexpr int64_t kBcmMaxM = 12;
constexpr int64_t kBcmMfmaMaxM = 48;

// The one-launch GEMV over the prepacked planes (gemv_q4_1_bcm): f16 A with
// 16-byte-aligned rows, K % 8 == 0.
inline bool bcm_ok(const NnopsGemmQ41Args& g)
{
    return g.b_soa && !g.trans_b && g.a_f16 && g.k % 8 == 0 && (g.lda % 8) == 0 && ((uintptr_t)g.a & 15) == 0;
}

inline bool kn_ring_ok(const NnopsGemmQ41Args& g)
{
    return !g.trans_b && g.a_f16 && g.k % 64 == 0 && (g.lda % 8) == 0 && ((uintptr_t)g.a & 15) == 0 &&
           (g.ldb_bytes % 16) == 0 && ((uintptr_t)g.b & 15) == 0 &&
           (g.b_soa ? 8 * g.ldb_bytes < INT32_MAX && 8 * g.ldb_dm * 4 < INT32_MAX : g.k * g.ldb_bytes < INT32_MAX);
}


// f32 A past the skinny and GEMV shapes, K % 64 == 0, either weight form
// (blocks along K: the ring; along N, raw rows or the prepacked planes: the
// kn ring): split into two f16 planes in the workspace (split_a_f32) and run
// the ring's SPLIT form (two f16 MFMAs per decoded weight fragment) instead
// of the f32 MFMA GEMM (config 4's shape at M = 512: 555 us on the f32
// matrix cores, 152 us split).
inline bool split_ok(const NnopsGemmQ41Args& g)
{
    if (g.a_f16 || g.k % 64 != 0 || skinny_ok(g) || use_gemv(g) || 4 * g.m * g.k >= INT32_MAX) {
        return false;
    }
    if (g.trans_b) {
        return !g.b_soa && 32 * g.ldb_bytes < INT32_MAX;
    }
    // blocks along N: the kn ring's weight conditions (its A is the planes)
    return (g.ldb_bytes % 16) == 0 && ((uintptr_t)g.b & 15) == 0 &&
           (g.b_soa ? 8 * g.ldb_bytes < INT32_MAX && 8 * g.ldb_dm * 4 < INT32_MAX : g.k * g.ldb_bytes < INT32_MAX);
}

inline size_t split_ws_bytes(const NnopsGemmQ41Args& g)
{
    return align_up((size_t)g.m * (size_t)g.k * 4) + align_up((size_t)g.m * 4);
}

// the prepacked planes' block-column pitches: nibbles in bytes, d|m in dwords
inline int64_t prepack_q41_nib_pitch(int64_t k) { return (k + 7) / 8 * 128; }
inline int64_t prepack_q41_dm_pitch(int64_t k) { return (k + 63) / 64 * 64; }

}  // namespace
}  // namespace nnops_amd

using namespace nnops_amd;

extern "C" size_t nnops_hip_gemm_q4_1_workspace_size(const NnopsGemmQ41Args* g)
{
    if (g != nullptr && split_ok(*g)) {
        return split_ws_bytes(*g);
    }
    if (g == nullptr || g->trans_b || !use_gemv(*g) || bcm_ok(*g)) {
        return 0;
    }
    // pointer alignment, which a size query may not see, picks between the
    // two blocks-along-N GEMVs: room for either
    const size_t split_bytes = align_up((size_t)kn_splits(*g) * (size_t)g->m * (size_t)g->n * sizeof(float));
    const KnDmaPlan kd = plan_kn_dma(*g);
    if (kd.groups > 0) {
        return std::max(split_bytes, align_up(kn_dma_part_bytes(kd)) + align_up((size_t)kd.groups * kd.splits * 8));
    }
    return split_bytes;
}

extern "C" int nnops_hip_gemm_q4_1(const NnopsGemmQ41Args* g, void* workspace, size_t ws_bytes, void* stream)
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
    if (g->out_kind != NNOPS_OUT_F32 && g->out_kind != NNOPS_OUT_F16) {
        return NNOPS_UNSUPPORTED;
    }
    if (g->m > INT32_MAX || g->n > INT32_MAX || g->k > INT32_MAX) {
        return NNOPS_UNSUPPORTED;
    }
    const int64_t nbn = (g->n + 31) / 32;
    // the prepacked planes' pitches are fixed by K (exact, checked below)
    const int64_t row_bytes = g->b_soa ? 0 : g->trans_b ? (g->k + 31) / 32 * 20 : nbn * 20;
    if (g->lda < g->k || g->ldc < g->n || g->ldb_bytes < row_bytes || (g->ldb_bytes & 3) ||
        ((uintptr_t)g->b & 3)) {
        return NNOPS_INVALID_ARGUMENT;
    }
    if (g->b_soa && (g->trans_b || g->b_dm == nullptr || g->ldb_bytes != prepack_q41_nib_pitch(g->k) ||
                     ((uintptr_t)g->b & 15) || ((uintptr_t)g->b_dm & 15) ||
                     g->ldb_dm != prepack_q41_dm_pitch(g->k))) {
        return NNOPS_INVALID_ARGUMENT;
    }
    const size_t need = nnops_hip_gemm_q4_1_workspace_size(g);
    if (need > 0 && (workspace == nullptr || ws_bytes < need)) {
        return NNOPS_NOT_INITIALIZED;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    Q41Kern k{};
    k.a = g->a;
    k.b = g->b;
    k.c = g->c;
    k.m = (int)g->m;
    k.n = (int)g->n;
    k.k = (int)g->k;
    k.lda = g->lda;
    k.ldc = g->ldc;
    k.ldb = g->ldb_bytes;
    k.out_f16 = g->out_kind == NNOPS_OUT_F16;
    k.bdm = g->b_soa ? g->b_dm : nullptr;
    k.ldbdm = g->b_soa ? g->ldb_dm : 0;
    const bool soa = g->b_soa != 0;

    if (skinny_ok(*g)) {
        // a few rows of A: the weight streams once per 16 rows
        for (int m0 = 0; m0 < k.m; m0 += 16) {
            Q41Kern kk = k;
            kk.m = std::min(16, k.m - m0);
            kk.a = static_cast<const char*>(g->a) + (int64_t)m0 * g->lda * (g->a_f16 ? 2 : 4);
            kk.c = static_cast<char*>(g->c) + (int64_t)m0 * g->ldc * (k.out_f16 ? 2 : 4);
            const dim3 grid((unsigned)((g->n + kSkRows - 1) / kSkRows));
            if (!g->a_f16) {
                NNOPS_LAUNCH(gemv_q4_1_skinny_f32<3>, grid, dim3(128), 0, s, kk);
            } else if (g->k % 512 == 0) {
                // two K halves per workgroup: four waves, two stages in flight
                NNOPS_LAUNCH((gemv_q4_1_skinny<2, 2>), grid, dim3(256), 0, s, kk);
            } else {
                NNOPS_LAUNCH((gemv_q4_1_skinny<4, 1>), grid, dim3(128), 0, s, kk);
            }
        }
    } else if (use_gemv(*g)) {
        // rows of A handled per pass: 2 (f16 pairs), 1 for f32 A
        const int mt = g->a_f16 ? 2 : 1;
        for (int m0 = 0; m0 < k.m; m0 += mt) {
            Q41Kern kk = k;
            kk.m = std::min(mt, k.m - m0);
            kk.a = static_cast<const char*>(g->a) + (int64_t)m0 * g->lda * (g->a_f16 ? 2 : 4);
            kk.c = static_cast<char*>(g->c) + (int64_t)m0 * g->ldc * (k.out_f16 ? 2 : 4);
            if (g->trans_b) {
                const unsigned blocks = (unsigned)((g->n + kNkWaves * kNkRowsPerWave - 1) / (kNkWaves * kNkRowsPerWave));
                if (g->a_f16) {
                    constexpr int R = 2;
                    const unsigned rb = (unsigned)((g->n + 4 * R - 1) / (4 * R));
                    const int64_t nbk = (g->k + 31) / 32;
                    // LDS-staged rows: whole 16-byte chunks per row, <= 128 blocks
                    const bool staged = nbk <= 128 && (nbk % 4) == 0 && (g->ldb_bytes % 16) == 0 &&
                                        ((uintptr_t)g->b & 15) == 0;
                    // K = 4096 rows stored back to back, aligned A: the pipelined form
                    const bool pipe = g->k == 128 * 32 && g->ldb_bytes == 128 * 20 && ((uintptr_t)g->b & 15) == 0 &&
                                      (g->lda % 8) == 0 && ((uintptr_t)kk.a & 15) == 0;
                    if (pipe) {
                        // 4 rows per wave: 10 KiB per wave in flight, one launch-wide wave of blocks
                        const unsigned rb4 = (unsigned)((g->n + 15) / 16);
                        if (kk.m == 1) {
                            NNOPS_LAUNCH((gemv_q4_1_pipe<1, 4>), dim3(rb4), dim3(256), 0, s, kk);
                        } else {
                            NNOPS_LAUNCH((gemv_q4_1_pipe<2, 4>), dim3(rb4), dim3(256), 0, s, kk);
                        }
                    } else if (staged) {
                        if (kk.m == 1) {
                            NNOPS_LAUNCH((gemv_q4_1_lds<1, R>), dim3(rb), dim3(256), 0, s, kk);
                        } else {
                            NNOPS_LAUNCH((gemv_q4_1_lds<2, R>), dim3(rb), dim3(256), 0, s, kk);
                        }
                    } else if (kk.m == 1) {
                        NNOPS_LAUNCH((gemv_q4_1_rows<1, R>), dim3(rb), dim3(256), 0, s, kk);
                    } else {
                        NNOPS_LAUNCH((gemv_q4_1_rows<2, R>), dim3(rb), dim3(256), 0, s, kk);
                    }
                } else {
                    NNOPS_LAUNCH((gemv_q4_1_nk<1, false>), dim3(blocks), dim3(256), 0, s, kk);
                }
            } else if (bcm_ok(*g)) {
                // the prepacked planes: one workgroup per block column, whole K
                // 8 waves, 4 chunks in flight per lane: 10.6 us at config 4
                // (4 waves x 2 chunks 12.0, 8 x 2 11.2, 4 x 8 10.8)
                if (kk.m == 1) {
                    NNOPS_LAUNCH((gemv_q4_1_bcm<1, 8, 4>), dim3((unsigned)nbn), dim3(512), 0, s, kk);
                } else {
                    NNOPS_LAUNCH((gemv_q4_1_bcm<2, 8, 4>), dim3((unsigned)nbn), dim3(512), 0, s, kk);
                }
            } else if (const KnDmaPlan pl = plan_kn_dma(*g); pl.groups > 0) {
                KnDma kd;
                kd.splits = pl.splits;
                kd.kper = pl.kper;
                kd.part = static_cast<float*>(workspace);
                kd.flag = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + align_up(kn_dma_part_bytes(pl)));
                kd.epoch = next_launch_epoch();
                const dim3 grid((unsigned)pl.groups, (unsigned)pl.splits);
                // 8 waves: four row-pair classes per stage hide the LDS and
                // dot latencies better than 4 (18.0 -> 17.0 us at config 4)
                if (kk.m == 1) {
                    NNOPS_LAUNCH((gemv_q4_1_kn_dma<1, 8>), grid, dim3(512), 0, s, kk, kd);
                } else {
                    NNOPS_LAUNCH((gemv_q4_1_kn_dma<2, 8>), grid, dim3(512), 0, s, kk, kd);
                }
            } else {
                kk.splits = kn_splits(*g);
                kk.partial = static_cast<float*>(workspace);
                const unsigned bx = (unsigned)(((g->n + 31) / 32 + 15) / 16);
                const dim3 grid(bx, kk.splits);
                if (g->a_f16 && kk.m == 1) {
                    if (soa) {
                        NNOPS_LAUNCH((gemv_q4_1_kn<1, true, true>), grid, dim3(256), 0, s, kk);
                    } else {
                        NNOPS_LAUNCH((gemv_q4_1_kn<1, true, false>), grid, dim3(256), 0, s, kk);
                    }
                } else if (g->a_f16) {
                    if (soa) {
                        NNOPS_LAUNCH((gemv_q4_1_kn<2, true, true>), grid, dim3(256), 0, s, kk);
                    } else {
                        NNOPS_LAUNCH((gemv_q4_1_kn<2, true, false>), grid, dim3(256), 0, s, kk);
                    }
                } else if (soa) {
                    NNOPS_LAUNCH((gemv_q4_1_kn<1, false, true>), grid, dim3(256), 0, s, kk);
                } else {
                    NNOPS_LAUNCH((gemv_q4_1_kn<1, false, false>), grid, dim3(256), 0, s, kk);
                }
                const int64_t total = (int64_t)kk.m * kk.n;
                if (kk.splits >= 32) {
                    NNOPS_LAUNCH(reduce_q4_1<16>, dim3((unsigned)((total * 16 + 255) / 256)), dim3(256), 0, s, kk);
                } else {
                    NNOPS_LAUNCH(reduce_q4_1<1>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, kk);
                }
            }
        }
    } else if (bcm_ok(*g) && g->m >= 3 && g->m <= kBcmMfmaMaxM && g->k % 256 == 0) {
        // a few rows of A over the prepacked planes on the matrix cores, the
        // weight streamed once per 16 rows
        for (int m0 = 0; m0 < k.m; m0 += 16) {
            Q41Kern kk = k;
            kk.m = std::min(16, k.m - m0);
            kk.a = static_cast<const char*>(g->a) + (int64_t)m0 * g->lda * 2;
            kk.c = static_cast<char*>(g->c) + (int64_t)m0 * g->ldc * (k.out_f16 ? 2 : 4);
            // 3 stages of 64 k in flight per wave (2 and 4 measured the same or slower;
            // so did A fragments loaded straight from L2, 8 waves per column, and
            // rotated K start points per workgroup: 12.6-19 us at M = 8)
            NNOPS_LAUNCH((gemv_q4_1_bcm_mfma<3>), dim3((unsigned)nbn), dim3(256), 0, s, kk);
        }
    } else if (bcm_ok(*g) && g->m <= kBcmMaxM) {
        // a few rows of A over the prepacked planes: the one-launch GEMV, up
        // to 8 rows per pass (its arithmetic grows with the rows: config 4's
        // shape 10.6 / 13.7 / 22.7 / 42.9 us for 1 / 2 / 4 / 8 rows, the ring
        // 77-85 us for any M up to 128)
        for (int m0 = 0; m0 < k.m;) {
            const int rem = k.m - m0;
            const int mt = rem > 4 ? 8 : rem > 2 ? 4 : 2;
            Q41Kern kk = k;
            kk.m = std::min(mt, rem);
            kk.a = static_cast<const char*>(g->a) + (int64_t)m0 * g->lda * 2;
            kk.c = static_cast<char*>(g->c) + (int64_t)m0 * g->ldc * (k.out_f16 ? 2 : 4);
            if (mt == 2) {
                NNOPS_LAUNCH((gemv_q4_1_bcm<2, 8, 4>), dim3((unsigned)nbn), dim3(512), 0, s, kk);
            } else if (mt == 4) {
                NNOPS_LAUNCH((gemv_q4_1_bcm<4, 8, 4>), dim3((unsigned)nbn), dim3(512), 0, s, kk);
            } else {
                NNOPS_LAUNCH((gemv_q4_1_bcm<8, 8, 2>), dim3((unsigned)nbn), dim3(512), 0, s, kk);
            }
            m0 += mt;
        }
    } else if (split_ok(*g)) {
        if (((uintptr_t)workspace & 15) != 0) {
            return NNOPS_INVALID_ARGUMENT;
        }
        _Float16* hi = static_cast<_Float16*>(workspace);
        _Float16* lo = hi + (int64_t)g->m * g->k;
        float* rs = reinterpret_cast<float*>(static_cast<char*>(workspace) + align_up((size_t)g->m * (size_t)g->k * 4));
        NNOPS_LAUNCH(split_a_f32, dim3((unsigned)g->m), dim3(256), 0, s, static_cast<const float*>(g->a), g->lda,
                     (int)g->k, hi, lo, rs);
        Q41Kern kk = k;
        kk.a = hi;
        kk.lda = g->k;
        kk.plane = g->m * g->k * 2;
        kk.row_scale = rs;
        const unsigned tiles = (unsigned)(((g->m + 127) / 128) * ((g->n + 255) / 256));
        if (g->trans_b && k.out_f16) {
            NNOPS_LAUNCH((gemm_q4_1_ring<true, 3, 1, 8, false, true>), dim3(tiles), dim3(512), 0, s, kk);
        } else if (g->trans_b) {
            NNOPS_LAUNCH((gemm_q4_1_ring<false, 3, 1, 8, false, true>), dim3(tiles), dim3(512), 0, s, kk);
        } else if (soa && k.out_f16) {
            NNOPS_LAUNCH((gemm_q4_1_kn_ring<true, 3, true, true>), dim3(tiles), dim3(512), 0, s, kk);
        } else if (soa) {
            NNOPS_LAUNCH((gemm_q4_1_kn_ring<false, 3, true, true>), dim3(tiles), dim3(512), 0, s, kk);
        } else if (k.out_f16) {
            NNOPS_LAUNCH((gemm_q4_1_kn_ring<true, 3, false, true>), dim3(tiles), dim3(512), 0, s, kk);
        } else {
            NNOPS_LAUNCH((gemm_q4_1_kn_ring<false, 3, false, true>), dim3(tiles), dim3(512), 0, s, kk);
        }
    } else if (!g->a_f16) {
        const unsigned tiles = (unsigned)(((g->m + 127) / 128) * ((g->n + 127) / 128));
        if (g->trans_b) {
            NNOPS_LAUNCH(gemm_q4_1_f32<0>, dim3(tiles), dim3(256), 0, s, k);
        } else if (soa) {
            NNOPS_LAUNCH(gemm_q4_1_f32<2>, dim3(tiles), dim3(256), 0, s, k);
        } else {
            NNOPS_LAUNCH(gemm_q4_1_f32<1>, dim3(tiles), dim3(256), 0, s, k);
        }
    } else if (g->trans_b && g->k % 64 == 0 && (g->lda % 8) == 0 && ((uintptr_t)g->a & 15) == 0) {
        // blocks along K: the ring kernel (A by DMA, B decoded in registers)
        const unsigned tiles = (unsigned)(((g->m + 127) / 128) * ((g->n + 255) / 256));
        // 8 waves (2 per SIMD), each 128 x 32: one wave's decode and stalls
        // overlap the other's matrix-core work, and no B row is decoded twice
        if (k.out_f16) {
            NNOPS_LAUNCH((gemm_q4_1_ring<true, 4, 1, 8>), dim3(tiles), dim3(512), 0, s, k);
        } else {
            NNOPS_LAUNCH((gemm_q4_1_ring<false, 4, 1, 8>), dim3(tiles), dim3(512), 0, s, k);
        }
    } else if (kn_ring_ok(*g)) {
        // blocks along N: the same ring, B rows staged raw and decoded per lane
        const unsigned tiles = (unsigned)(((g->m + 127) / 128) * ((g->n + 255) / 256));
        if (k.out_f16) {
            if (soa) {
                NNOPS_LAUNCH((gemm_q4_1_kn_ring<true, 4, true>), dim3(tiles), dim3(512), 0, s, k);
            } else {
                NNOPS_LAUNCH((gemm_q4_1_kn_ring<true, 4, false>), dim3(tiles), dim3(512), 0, s, k);
            }
        } else if (soa) {
            NNOPS_LAUNCH((gemm_q4_1_kn_ring<false, 4, true>), dim3(tiles), dim3(512), 0, s, k);
        } else {
            NNOPS_LAUNCH((gemm_q4_1_kn_ring<false, 4, false>), dim3(tiles), dim3(512), 0, s, k);
        }
    } else {
        const unsigned tiles = (unsigned)(((g->m + 127) / 128) * ((g->n + 127) / 128));
        if (g->trans_b) {
            NNOPS_LAUNCH((gemm_q4_1_mfma<128, 128, 2, 2, true>), dim3(tiles), dim3(256), 0, s, k);
        } else if (soa) {
            NNOPS_LAUNCH((gemm_q4_1_mfma<128, 128, 2, 2, false, true>), dim3(tiles), dim3(256), 0, s, k);
        } else {
            NNOPS_LAUNCH((gemm_q4_1_mfma<128, 128, 2, 2, false>), dim3(tiles), dim3(256), 0, s, k);
        }
    }
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}

extern "C" int nnops_hip_gemm_q4_1_fused(const NnopsGemmQ41Args* g, const NnopsFpOutArgs* pass, void* stream)
{
    const TimingDisarm disarm;
    if (g == nullptr || pass == nullptr) {
        return NNOPS_INVALID_ARGUMENT;
    }
    // the blocks-along-K ring route (f16 A past the GEMV and skinny shapes)
    // and, gated, the pipelined GEMV (M <= 2, K = 4096, rows back to back);
    // anything else is the caller's two-step form
    if (!g->trans_b || g->b_soa || !g->a_f16 || g->m <= 0 || g->n <= 0 || g->k <= 0 || g->m > INT32_MAX ||
        g->n > INT32_MAX || g->k > INT32_MAX || g->a == nullptr || g->b == nullptr || g->lda < g->k ||
        g->ldb_bytes < (g->k + 31) / 32 * 20 || (g->ldb_bytes & 3) || ((uintptr_t)g->b & 3)) {
        return NNOPS_UNSUPPORTED;
    }
    const bool pipe_gemv = g->m <= 2 && g->k == 128 * 32 && g->ldb_bytes == 128 * 20 && ((uintptr_t)g->b & 15) == 0 &&
                           (g->lda % 8) == 0 && ((uintptr_t)g->a & 15) == 0 && pass->gated && g->n % 2 == 0;
    if (!pipe_gemv && (use_gemv(*g) || skinny_ok(*g) || g->k % 64 != 0 || (g->lda % 8) != 0 ||
                       ((uintptr_t)g->a & 15) != 0)) {
        return NNOPS_UNSUPPORTED;
    }
    FpOut fo;
    if (const int rc = make_fp_out(pass, fo); rc != NNOPS_OK) {
        return rc;
    }
    if (pass->rows != g->m || pass->n * (pass->gated ? 2 : 1) != g->n) {
        return NNOPS_INVALID_ARGUMENT;
    }
    // only the gated form gains: the plain pass's arithmetic in the GEMM's
    // write-back costs more than the staging it saves
    if (!pass->gated) {
        return NNOPS_UNSUPPORTED;
    }
    // the gated tile addresses both halves of the weight from its start
    if (pass->gated && g->n * g->ldb_bytes >= INT32_MAX) {
        return NNOPS_UNSUPPORTED;
    }
    Q41Kern k{};
    k.a = g->a;
    k.b = g->b;
    k.m = (int)g->m;
    k.n = (int)g->n;
    k.k = (int)g->k;
    k.lda = g->lda;
    k.ldb = g->ldb_bytes;
    k.fo = fo;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (pipe_gemv) {
        // two outputs per wave, four waves per workgroup
        const unsigned rb = (unsigned)((pass->n + 7) / 8);
        if (g->m == 1) {
            if (fo.out_f16) {
                NNOPS_LAUNCH((gemv_q4_1_pipe<1, 4, true, true>), dim3(rb), dim3(256), 0, s, k);
            } else {
                NNOPS_LAUNCH((gemv_q4_1_pipe<1, 4, true, false>), dim3(rb), dim3(256), 0, s, k);
            }
        } else {
            if (fo.out_f16) {
                NNOPS_LAUNCH((gemv_q4_1_pipe<2, 4, true, true>), dim3(rb), dim3(256), 0, s, k);
            } else {
                NNOPS_LAUNCH((gemv_q4_1_pipe<2, 4, true, false>), dim3(rb), dim3(256), 0, s, k);
            }
        }
        return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
    }
    const int64_t tiles_m = (g->m + 127) / 128;
    const unsigned tiles = (unsigned)(tiles_m * ((pass->n + 127) / 128));
    NNOPS_LAUNCH((gemm_q4_1_ring<false, 4, 1, 8, true>), dim3(tiles), dim3(512), 0, s, k);
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}

extern "C" size_t nnops_hip_prepack_q4_1_bytes(int64_t k, int64_t n)
{
    if (k <= 0 || n <= 0) {
        return 0;
    }
    const size_t nbn = (size_t)((n + 31) / 32);
    return align_up(nbn * (size_t)prepack_q41_nib_pitch(k)) + nbn * (size_t)prepack_q41_dm_pitch(k) * 4;
}

extern "C" int nnops_hip_prepack_q4_1(const uint8_t* b, int64_t k, int64_t n, int64_t ldb_bytes, int32_t trans_b,
                                      void* out, void* stream)
{
    const TimingDisarm disarm;
    if (trans_b) {
        return NNOPS_UNSUPPORTED;  // blocks along K: no packed form
    }
    if (b == nullptr || out == nullptr || k <= 0 || n <= 0 || k > INT32_MAX || n > INT32_MAX) {
        return NNOPS_INVALID_ARGUMENT;
    }
    const int64_t nbn = (n + 31) / 32;
    if (ldb_bytes < nbn * 20 || (ldb_bytes & 3) || ((uintptr_t)b & 3) || ((uintptr_t)out & 255)) {
        return NNOPS_INVALID_ARGUMENT;
    }
    uint8_t* nib = static_cast<uint8_t*>(out);
    uint32_t* dm = reinterpret_cast<uint32_t*>(nib + align_up((size_t)nbn * (size_t)prepack_q41_nib_pitch(k)));
    const int64_t blocks = k * nbn;
    NNOPS_LAUNCH(prepack_q4_1_kn, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), b, ldb_bytes, (int)k, (int)nbn, nib, dm,
                       prepack_q41_dm_pitch(k));
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}

extern "C" const char* nnops_hip_build_info(void)
{
    return "nnops_amd gfx950 (hand-written HIP: int8 MFMA GEMM/GEMV, Q4_1 GEMV/MFMA GEMM)";
}

extern "C" int nnops_hip_time_next_launch(void* start_event, void* stop_event)
{
    if ((start_event == nullptr) != (stop_event == nullptr)) {
        return NNOPS_INVALID_ARGUMENT;
    }
    nnops_amd::launch_timing() = nnops_amd::LaunchTiming{static_cast<hipEvent_t>(start_event),
                                                         static_cast<hipEvent_t>(stop_event)};
    return NNOPS_OK;
}
