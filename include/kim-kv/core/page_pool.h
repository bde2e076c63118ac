// Slot/generation page pool with a LIFO free list
// (include/kim-kv/core/page_pool.h of the reference).
#pragma once

#include "kim-kv/core/page_handle.h"
#include "kim-kv/core/page_types.h"

#include <cstdint>
#include <mutex>
#include <vector>

namespace kimkvcache {

struct PageAllocationResult final {
    PagePoolError error{PagePoolError::None};
    PageHandle handle{PageHandle::invalid()};

    [[nodiscard]] constexpr bool ok() const noexcept { return error == PagePoolError::None; }
    [[nodiscard]] explicit constexpr operator bool() const noexcept { return ok(); }
};

struct PagePoolSnapshot final {
    PageKind kind{PageKind::Micro};
    std::uint32_t total_slots{0};
    std::uint32_t free_slots{0};
    std::uint32_t allocated_slots{0};
    std::uint64_t successful_allocations{0};
    std::uint64_t successful_releases{0};
    std::uint64_t failed_allocations{0};
    std::uint64_t rejected_releases{0};

    [[nodiscard]] constexpr bool capacityBalanced() const noexcept
    {
        return total_slots == free_slots + allocated_slots;
    }
};

// Thread-safe.  Exhaustion and bad releases are reported as errors, never
// thrown; only corrupted internal state throws std::logic_error.
class PagePool final {
public:
    PagePool(PageKind kind, std::uint32_t capacity);

    PagePool(PagePool const&) = delete;
    PagePool& operator=(PagePool const&) = delete;
    PagePool(PagePool&&) = delete;
    PagePool& operator=(PagePool&&) = delete;

    [[nodiscard]] PageKind kind() const noexcept { return kind_; }
    [[nodiscard]] std::uint32_t capacity() const noexcept { return capacity_; }

    [[nodiscard]] PageAllocationResult allocate();
    [[nodiscard]] PagePoolError release(PageHandle handle);
    [[nodiscard]] PagePoolError validate(PageHandle handle) const;
    [[nodiscard]] PagePoolSnapshot snapshot() const;
    [[nodiscard]] bool checkInvariants() const;

private:
    struct Slot final {
        std::uint32_t generation{0};
        bool allocated{false};
    };

    [[nodiscard]] PagePoolError validateLocked(PageHandle handle) const noexcept;

    PageKind kind_;
    std::uint32_t capacity_;
    std::vector<Slot> slots_;
    std::vector<std::uint32_t> free_;   // back() is the next slot handed out
    std::uint32_t allocated_{0};
    std::uint64_t allocations_{0};
    std::uint64_t releases_{0};
    std::uint64_t failed_allocations_{0};
    std::uint64_t rejected_releases_{0};
    mutable std::mutex mutex_;
};

}  // namespace kimkvcache
