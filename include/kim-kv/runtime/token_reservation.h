// Single-token reservation result (include/kim-kv/runtime/token_reservation.h of the reference).
#pragma once

#include "kim-kv/core/block_table.h"
#include "kim-kv/core/page_state.h"
#include "kim-kv/runtime/promotion.h"

#include <cstdint>

namespace kimkvcache {

using KvTokenReservationId = std::uint64_t;
constexpr KvTokenReservationId kInvalidKvTokenReservationId = 0;

// `before` stays the visible table until commit; `reserved` is the candidate
// table including the uncommitted token, visible only to its transaction.
struct TokenReservationResult final {
    KvCacheError error{KvCacheError::None};
    KvTokenReservationId reservation_id{kInvalidKvTokenReservationId};
    RequestId request_id{kInvalidRequestId};
    std::uint32_t logical_token_position{0};
    BlockTable before{};
    BlockTable reserved{};

    [[nodiscard]] constexpr bool ok() const noexcept
    {
        return error == KvCacheError::None && reservation_id != kInvalidKvTokenReservationId;
    }
    [[nodiscard]] explicit constexpr operator bool() const noexcept { return ok(); }
};

}  // namespace kimkvcache
