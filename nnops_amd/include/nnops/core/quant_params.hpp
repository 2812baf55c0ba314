#pragma once
/// @file quant_params.hpp
/// @brief QuantParams — scale / zero point of an integer tensor, non-owning.
///
/// Field-for-field nnops' struct (include/nnops/core/quant_params.hpp:36-61):
/// PerTensor uses the scalars, PerToken one pair per row, PerChannel one pair
/// per channel of the op's channel axis (MatMul: output column). The arrays may
/// live in host memory (the HIP backend stages them into the workspace, as
/// nnops' CUDA backend stages them) or in device memory (read in place).

#include <cstdint>

namespace nnops {

enum class QuantGranularity : uint8_t {
    PerTensor = 0,
    PerToken = 1,
    PerChannel = 2,
};

struct QuantParams {
    QuantGranularity granularity = QuantGranularity::PerTensor;
    float scale = 1.0f;
    int32_t zero_point = 0;
    const float* scale_data = nullptr;
    const int32_t* zero_point_data = nullptr;
    int64_t num_scales = 0;

    bool is_active() const noexcept
    {
        if (scale_data != nullptr || zero_point_data != nullptr) {
            return true;
        }
        return scale != 1.0f || zero_point != 0;
    }
};

}  // namespace nnops
