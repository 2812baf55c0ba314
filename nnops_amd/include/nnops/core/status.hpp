#pragma once
/// @file status.hpp
/// @brief Status — the error code every fallible entry point returns.
///
/// Same values and meaning as nnops::Status (include/nnops/core/status.hpp:19-33
/// in the nnops tree), so a caller's error handling carries over unchanged. A
/// rejected call writes nothing to its outputs.

#include <cstdint>

namespace nnops {

enum class Status : uint8_t {
    ok = 0,
    invalid_argument,   ///< malformed call: counts, ranks, shapes, dtypes
    unsupported,        ///< well-formed, but this backend has no route for it
    not_initialized,    ///< required state absent: workspace missing or too small
    out_of_memory,
    internal,           ///< a library invariant failed, or a launch failed
};

constexpr bool is_ok(Status s) noexcept { return s == Status::ok; }
constexpr bool is_error(Status s) noexcept { return s != Status::ok; }

inline const char* to_string(Status s) noexcept
{
    switch (s) {
    case Status::ok: return "ok";
    case Status::invalid_argument: return "invalid_argument";
    case Status::unsupported: return "unsupported";
    case Status::not_initialized: return "not_initialized";
    case Status::out_of_memory: return "out_of_memory";
    case Status::internal: return "internal";
    }
    return "unknown";
}

}  // namespace nnops
