// Q4_1 codec on gfx950: f32/f16 rows -> llama.cpp block_q4_1 rows, and back.
//
// quantize   nnops' quantize_q4 (include/nnops/detail/q4_1.hpp:92-149), which
//            is llama.cpp's quantize_row_q4_1_ref: per block of 32 values the
//            block's own min and max give d = (max - min) / 15 and m = min (both
//            stored as f16, nearest even), each value becomes
//            q = min(trunc((x - min) * (1 / d) + 0.5), 15) (1 / d = 0 when
//            d = 0), low nibble of byte j = value j, high nibble = value j + 16.
//            The f32 arithmetic is the reference's operation for operation
//            (separately rounded; d and 1 / d from the f32 min / max, before
//            the f16 store), so the blocks are byte-identical.
// dequantize nnops' pack_q4 (q4_1.hpp:155-183): y = d * q + m in f32 (d * q is
//            exact for an f16 d and q <= 15, so this is one rounding), f16
//            output rounded to nearest even at the store.
//
// Both are load-time passes over a weight, bound by HBM. Eight lanes share a
// block: lane l of the eight owns values 4l .. 4l + 3, so a wave reads 8
// blocks' 256 consecutive values per load; min / max are combined across the
// eight lanes with xor shuffles, and the low / high nibble halves meet with
// one more (lane l and l + 4). A partial last block of a row takes d and m
// from the values that exist and leaves the missing nibbles zero (nnops does
// the same); rows are independent (ld_src / ld_dst pitches).
#include "common.hpp"

namespace nnops_amd {
namespace {

struct CodecArgs {
    const void* src;
    void* dst;
    int64_t rows, cols;
    int64_t ld_src;     // quantize: source row stride in elements; dequantize: bytes
    int64_t ld_dst;     // quantize: block-row pitch in bytes; dequantize: elements
    int32_t f16;        // the float side is f16 (else f32)
    int64_t nb;         // blocks per row
};

__device__ __forceinline__ float load_val(const void* p, int64_t i, bool f16)
{
    if (f16) {
        return (float)static_cast<const _Float16*>(p)[i];
    }
    return static_cast<const float*>(p)[i];
}

__device__ __forceinline__ uint32_t f16_bits(float v)
{
    const _Float16 h = (_Float16)v;   // round to nearest even
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

__global__ __launch_bounds__(256) void q4_1_quantize_kernel(CodecArgs p)
{
    const int64_t gid = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    const int l = threadIdx.x & 7;
    const bool live = gid < p.rows * p.nb;
    const int64_t row = live ? gid / p.nb : 0;
    const int64_t b = live ? gid - row * p.nb : 0;
    const int64_t base = b * 32;
    const int n = live ? (int)min((int64_t)32, p.cols - base) : 0;
    const bool f16 = p.f16 != 0;
    const int64_t off = row * p.ld_src + base;

    float x[4];
    float lo = __builtin_inff(), hi = -__builtin_inff();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int j = 4 * l + e;
        x[e] = j < n ? load_val(p.src, off + j, f16) : 0.0f;
        if (j < n) {
            lo = x[e] < lo ? x[e] : lo;
            hi = x[e] > hi ? x[e] : hi;
        }
    }
    // min / max over the block's eight lanes (lanes of one block are an
    // aligned group of 8, so xor 1, 2, 4 stay inside it)
#pragma unroll
    for (int s = 1; s < 8; s <<= 1) {
        const float olo = __shfl_xor(lo, s, 64);
        const float ohi = __shfl_xor(hi, s, 64);
        lo = olo < lo ? olo : lo;
        hi = ohi > hi ? ohi : hi;
    }
    const float d = __fdiv_rn(__fsub_rn(hi, lo), 15.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint32_t q4 = 0;   // this lane's 4 nibbles, one per byte
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int j = 4 * l + e;
        uint32_t q = 0;
        if (j < n) {
            const float qf = __fadd_rn(__fmul_rn(__fsub_rn(x[e], lo), id), 0.5f);
            q = qf < 15.0f ? (uint32_t)(int)qf : 15u;
        }
        q4 |= q << (8 * e);
    }
    // byte j = value j | value (j + 16) << 4: lane l < 4 holds values
    // 4l .. 4l + 3 and takes 16 + 4l .. from lane l + 4, which makes nibble
    // dword l; lane 4 stores d | m (dwords of the 20-byte block: 0 = d|m,
    // 1 .. 4 = nibbles)
    const uint32_t up = (uint32_t)__shfl_xor((int)q4, 4, 64);
    if (!live || l > 4) {
        return;
    }
    uint32_t* blk = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(p.dst) + row * p.ld_dst + b * 20);
    if (l == 4) {
        blk[0] = f16_bits(d) | (f16_bits(lo) << 16);
    } else {
        blk[1 + l] = q4 | (up << 4);
    }
}

__global__ __launch_bounds__(256) void q4_1_dequantize_kernel(CodecArgs p)
{
    const int64_t gid = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    const int l = threadIdx.x & 7;
    if (gid >= p.rows * p.nb) {
        return;
    }
    const int64_t row = gid / p.nb;
    const int64_t b = gid - row * p.nb;
    const uint8_t* blk = static_cast<const uint8_t*>(p.src) + row * p.ld_src + b * 20;
    const uint32_t dm = *reinterpret_cast<const uint32_t*>(blk);
    const uint32_t qs = *reinterpret_cast<const uint32_t*>(blk + 4 + 4 * (l & 3));
    _Float16 dh, mh;
    const uint16_t db = (uint16_t)(dm & 0xffffu), mb = (uint16_t)(dm >> 16);
    __builtin_memcpy(&dh, &db, 2);
    __builtin_memcpy(&mh, &mb, 2);
    const float d = (float)dh, m = (float)mh;
    const int shift = (l >> 2) * 4;
    const int64_t base = b * 32 + 4 * l;
    const int n = (int)min((int64_t)4, p.cols - base);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (e < n) {
            const float q = (float)((qs >> (8 * e + shift)) & 15u);
            const float y = __fadd_rn(__fmul_rn(d, q), m);
            const int64_t i = row * p.ld_dst + base + e;
            if (p.f16) {
                static_cast<_Float16*>(p.dst)[i] = (_Float16)y;
            } else {
                static_cast<float*>(p.dst)[i] = y;
            }
        }
    }
}

int check_codec(const void* src, const void* dst, int64_t rows, int64_t cols)
{
    if (rows < 0 || cols < 0) {
        return NNOPS_INVALID_ARGUMENT;
    }
    if (rows > 0 && cols > 0 && (src == nullptr || dst == nullptr)) {
        return NNOPS_INVALID_ARGUMENT;
    }
    return NNOPS_OK;
}

unsigned codec_grid(int64_t blocks) { return (unsigned)((blocks + 31) / 32); }

// 32 blocks per 256-thread workgroup: the grid's work-items must fit a
// dispatch's 32-bit count.
bool codec_grid_fits(int64_t blocks) { return (blocks + 31) / 32 <= (int64_t)(UINT32_MAX / 256); }

}  // namespace
}  // namespace nnops_amd

using namespace nnops_amd;

extern "C" int nnops_hip_q4_1_quantize(const void* src, int32_t src_f16, int64_t rows, int64_t cols, int64_t ld_src,
                                       void* dst, int64_t ld_dst_bytes, void* stream)
{
    const TimingDisarm disarm;
    if (int rc = check_codec(src, dst, rows, cols); rc != NNOPS_OK) {
        return rc;
    }
    if (rows == 0 || cols == 0) {
        return NNOPS_OK;
    }
    const int64_t nb = (cols + 31) / 32;
    const size_t esz = src_f16 ? 2 : 4;
    if (ld_src < cols || ld_dst_bytes < nb * 20 || (ld_dst_bytes & 3) || ((uintptr_t)dst & 3) ||
        ((uintptr_t)src % esz) != 0) {
        return NNOPS_INVALID_ARGUMENT;
    }
    if (!codec_grid_fits(rows * nb)) {
        return NNOPS_UNSUPPORTED;   // one dispatch holds at most 2^32 - 1 work-items
    }
    CodecArgs a{src, dst, rows, cols, ld_src, ld_dst_bytes, src_f16 ? 1 : 0, nb};
    NNOPS_LAUNCH(q4_1_quantize_kernel, dim3(codec_grid(rows * nb)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), a);
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}

extern "C" int nnops_hip_q4_1_dequantize(const void* src, int64_t ld_src_bytes, int64_t rows, int64_t cols, void* dst,
                                         int32_t dst_f16, int64_t ld_dst, void* stream)
{
    const TimingDisarm disarm;
    if (int rc = check_codec(src, dst, rows, cols); rc != NNOPS_OK) {
        return rc;
    }
    if (rows == 0 || cols == 0) {
        return NNOPS_OK;
    }
    const int64_t nb = (cols + 31) / 32;
    const size_t esz = dst_f16 ? 2 : 4;
    if (ld_dst < cols || ld_src_bytes < nb * 20 || (ld_src_bytes & 3) || ((uintptr_t)src & 3) ||
        ((uintptr_t)dst % esz) != 0) {
        return NNOPS_INVALID_ARGUMENT;
    }
    if (!codec_grid_fits(rows * nb)) {
        return NNOPS_UNSUPPORTED;   // one dispatch holds at most 2^32 - 1 work-items
    }
    CodecArgs a{src, dst, rows, cols, ld_src_bytes, ld_dst, dst_f16 ? 1 : 0, nb};
    NNOPS_LAUNCH(q4_1_dequantize_kernel, dim3(codec_grid(rows * nb)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), a);
    return hipGetLastError() == hipSuccess ? NNOPS_OK : NNOPS_INTERNAL;
}
