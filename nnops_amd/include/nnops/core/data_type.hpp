#pragma once
/// @file data_type.hpp
/// @brief DataType and its storage helpers.
///
/// The enum values are nnops' (include/nnops/core/data_type.hpp:23-36) so a
/// descriptor built by an nnops caller means the same here. q4_1 is llama.cpp's
/// block format: 32 values in a 20-byte block (f16 d, f16 m, 16 nibble bytes),
/// value = d*q + m; it has no per-element size, so row sizes go through
/// data_type_row_bytes() and strides through data_type_stride_unit().

#include <cstddef>
#include <cstdint>

namespace nnops {

enum class DataType : uint8_t {
    f32 = 0,
    f16 = 1,
    bf16 = 2,
    s8 = 3,
    u8 = 4,
    s32 = 5,
    s64 = 6,
    f8_e4m3 = 7,
    f8_e5m2 = 8,
    s4 = 9,
    u4 = 10,
    q4_1 = 11,
};

inline constexpr int64_t q4_1_block_elems = 32;
inline constexpr size_t q4_1_block_bytes = 20;

constexpr size_t data_type_size(DataType dt) noexcept
{
    switch (dt) {
    case DataType::f32: return 4;
    case DataType::f16: return 2;
    case DataType::bf16: return 2;
    case DataType::s8: return 1;
    case DataType::u8: return 1;
    case DataType::s32: return 4;
    case DataType::s64: return 8;
    case DataType::f8_e4m3: return 1;
    case DataType::f8_e5m2: return 1;
    case DataType::s4:
    case DataType::u4:
    case DataType::q4_1: return 0;
    }
    return 0;
}

constexpr bool is_block_packed_dtype(DataType dt) noexcept { return dt == DataType::q4_1; }

/// One row step: the element size, or the 20-byte block for q4_1.
constexpr size_t data_type_stride_unit(DataType dt) noexcept
{
    return is_block_packed_dtype(dt) ? q4_1_block_bytes : data_type_size(dt);
}

/// Bytes of a row of `cols` elements (q4_1 rounds up to whole blocks).
constexpr size_t data_type_row_bytes(DataType dt, int64_t cols) noexcept
{
    if (cols <= 0) {
        return 0;
    }
    if (is_block_packed_dtype(dt)) {
        return static_cast<size_t>((cols + q4_1_block_elems - 1) / q4_1_block_elems) * q4_1_block_bytes;
    }
    if (dt == DataType::s4 || dt == DataType::u4) {
        return static_cast<size_t>((cols + 1) / 2);
    }
    return static_cast<size_t>(cols) * data_type_size(dt);
}

constexpr bool is_quantized_dtype(DataType dt) noexcept
{
    return dt == DataType::s8 || dt == DataType::u8 || dt == DataType::s4 || dt == DataType::u4;
}

}  // namespace nnops
