#pragma once
/// @file backend.hpp
/// @brief Backend selector. The values of nnops' enum (include/nnops/core/
/// backend.hpp:16-21) are kept and HIP is appended, the enum being append-only.

#include <cstdint>

namespace nnops {

enum class Backend : uint8_t {
    CPU = 0,
    CUDA = 1,
    Vulkan = 2,
    Metal = 3,
    HIP = 4,  ///< AMD Instinct MI355X (gfx950): the backend this library implements
};

}  // namespace nnops
