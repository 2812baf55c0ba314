#pragma once
/// @file compute_context.hpp
/// @brief ComputeContext — per-call execution parameters.
///
/// nnops' context (include/nnops/core/compute_context.hpp:24-48) carries an
/// opaque `cuda_stream`; the HIP backend reads `hip_stream` (a hipStream_t,
/// nullptr = the null stream) the same way. Work is enqueued on it and
/// compute() returns without synchronising.

#include "nnops/core/backend.hpp"

namespace nnops {

struct ComputeContext {
    Backend expected_backend = Backend::HIP;  ///< informational
    void* cuda_stream = nullptr;              ///< kept for source compatibility; unused
    void* hip_stream = nullptr;               ///< hipStream_t, opaque
};

}  // namespace nnops
