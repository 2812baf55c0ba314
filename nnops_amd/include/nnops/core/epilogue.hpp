#pragma once
/// @file epilogue.hpp
/// @brief Epilogue — the activation / clip / quantization stage fused into an
/// operator's write-back. Same enum values and fields as nnops
/// (include/nnops/core/epilogue.hpp:22-92).

#include <cstdint>
#include <limits>

namespace nnops {

enum class EpilogueActivateType : uint8_t {
    None = 0,
    Relu = 1,
    Gelu = 2,
    Sigmoid = 3,
    Tanh = 4,
    LeakyRelu = 5,
    Silu = 6,
    HardSwish = 7,
    Elu = 8,
    Relu6 = 9,
};

enum class EpilogueQuantType : uint8_t {
    None = 0,
    Requantize = 1,  ///< y = clamp(round(x / scale) + zero_point)
    Dequantize = 2,
};

struct Epilogue {
    EpilogueActivateType type = EpilogueActivateType::None;
    float alpha = 0.0f;
    float beta = 1.0f;
    float min_clip = -std::numeric_limits<float>::infinity();
    float max_clip = std::numeric_limits<float>::infinity();

    EpilogueQuantType quant = EpilogueQuantType::None;
    /// One entry per output row when quant_param_count > 1, else per tensor.
    const float* quant_scales = nullptr;
    const int32_t* quant_zero_points = nullptr;
    int64_t quant_param_count = 0;
    int64_t quant_axis = 0;
};

inline bool epilogue_is_active(const Epilogue& ep) noexcept
{
    return ep.type != EpilogueActivateType::None || ep.quant != EpilogueQuantType::None ||
           ep.min_clip > -std::numeric_limits<float>::infinity() ||
           ep.max_clip < std::numeric_limits<float>::infinity();
}

}  // namespace nnops
