// Device status types of the HIP backend; counterpart of the reference's
// include/kim-kv/cuda/cuda_status.h (same enumerators and meaning).
#pragma once

#include "kim-kv/core/page_state.h"

#include <cstddef>
#include <cstdint>
#include <string_view>

namespace kimkvcache {

// Opaque hipStream_t; nullptr is the device's default stream.
using HipStream = void*;

struct HipStorageSnapshot final {
    std::uint32_t micro_capacity{0};
    std::uint32_t extent_capacity{0};
    std::uint16_t micro_page_tokens{kMicroPageTokenCapacity};
    std::uint16_t extent_page_tokens{kExtentPageTokenCapacity};
    std::size_t micro_reserved_bytes{0};
    std::size_t extent_reserved_bytes{0};

    [[nodiscard]] constexpr std::size_t totalReservedBytes() const noexcept
    {
        return micro_reserved_bytes + extent_reserved_bytes;
    }
};

enum class HipError : std::uint8_t {
    None,
    InvalidArgument,
    RuntimeUnavailable,
    AllocationFailed,
    SubmissionFailed,
    NotReady,
    ExecutionFailed,
    InternalError,
};

[[nodiscard]] constexpr std::string_view toString(HipError error) noexcept
{
    switch (error) {
    case HipError::None: return "none";
    case HipError::InvalidArgument: return "invalid_argument";
    case HipError::RuntimeUnavailable: return "runtime_unavailable";
    case HipError::AllocationFailed: return "allocation_failed";
    case HipError::SubmissionFailed: return "submission_failed";
    case HipError::NotReady: return "not_ready";
    case HipError::ExecutionFailed: return "execution_failed";
    case HipError::InternalError: return "internal_error";
    }
    return "unknown";
}

struct HipStatus final {
    HipError error{HipError::None};
    int native_error{0};

    [[nodiscard]] constexpr bool ok() const noexcept { return error == HipError::None; }
    [[nodiscard]] explicit constexpr operator bool() const noexcept { return ok(); }
};

// Deterministic one-shot fault hooks (CudaFailurePoint in the reference).
enum class HipFailurePoint : std::uint8_t {
    Submission,
    Completion,
};

}  // namespace kimkvcache
