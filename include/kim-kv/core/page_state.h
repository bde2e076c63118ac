// Page capacities, page states and KvCacheError
// (include/kim-kv/core/page_state.h of the reference).
#pragma once

#include "kim-kv/core/page_types.h"

#include <cstdint>
#include <string_view>

namespace kimkvcache {

constexpr std::uint16_t kMicroPageTokenCapacity = 8;
constexpr std::uint16_t kExtentPageTokenCapacity = 64;

[[nodiscard]] constexpr std::uint16_t pageTokenCapacity(PageKind kind) noexcept
{
    return kind == PageKind::Micro ? kMicroPageTokenCapacity
        : kind == PageKind::Extent ? kExtentPageTokenCapacity
                                   : 0;
}

// Life cycle of a physical page as seen by KvCacheManager.
enum class PageState : std::uint8_t {
    Free,        // on the pool's free list
    Mutable,     // partial micro tail owned by exactly one request
    Sealed,      // immutable; may be shared by forks
    CopyTarget,  // allocated, being written, not yet visible in any table
    Retiring,    // unreferenced but still pinned or leased
};

[[nodiscard]] constexpr std::string_view toString(PageState state) noexcept
{
    switch (state) {
    case PageState::Free: return "free";
    case PageState::Mutable: return "mutable";
    case PageState::Sealed: return "sealed";
    case PageState::CopyTarget: return "copy_target";
    case PageState::Retiring: return "retiring";
    }
    return "unknown";
}

enum class KvCacheError : std::uint8_t {
    None,
    InvalidArgument,
    RequestNotFound,
    RequestAlreadyExists,
    RequestConflict,
    ResourceExhausted,
    InvalidState,
    TokenReservationNotFound,
    PromotionNotEligible,
    PromotionNotFound,
    PromotionConflict,
    InternalInvariantViolation,
};

[[nodiscard]] constexpr std::string_view toString(KvCacheError error) noexcept
{
    switch (error) {
    case KvCacheError::None: return "none";
    case KvCacheError::InvalidArgument: return "invalid_argument";
    case KvCacheError::RequestNotFound: return "request_not_found";
    case KvCacheError::RequestAlreadyExists: return "request_already_exists";
    case KvCacheError::RequestConflict: return "request_conflict";
    case KvCacheError::ResourceExhausted: return "resource_exhausted";
    case KvCacheError::InvalidState: return "invalid_state";
    case KvCacheError::TokenReservationNotFound: return "token_reservation_not_found";
    case KvCacheError::PromotionNotEligible: return "promotion_not_eligible";
    case KvCacheError::PromotionNotFound: return "promotion_not_found";
    case KvCacheError::PromotionConflict: return "promotion_conflict";
    case KvCacheError::InternalInvariantViolation: return "internal_invariant_violation";
    }
    return "unknown";
}

}  // namespace kimkvcache
