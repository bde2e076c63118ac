// Page leases: keep physical pages alive across asynchronous device access
// (include/kim-kv/runtime/page_lease.h of the reference).  While a lease holds
// a page, losing its last table reference only moves it to Retiring; it
// returns to the pool when the lease is released.
#pragma once

#include "kim-kv/core/block_table.h"
#include "kim-kv/core/page_state.h"

#include <cstdint>
#include <vector>

namespace kimkvcache {

using PageLeaseId = std::uint64_t;
constexpr PageLeaseId kInvalidPageLeaseId = 0;

struct PageLeaseAcquireResult final {
    KvCacheError error{KvCacheError::None};
    PageLeaseId lease_id{kInvalidPageLeaseId};
    BlockTable table{};
    std::vector<PageHandle> handles{};

    [[nodiscard]] bool ok() const noexcept { return error == KvCacheError::None; }
    [[nodiscard]] explicit operator bool() const noexcept { return ok(); }
};

}  // namespace kimkvcache
