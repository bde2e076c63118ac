// Per-request page table: ordered, contiguous mapping entries
// (include/kim-kv/core/block_table.h of the reference).
#pragma once

#include "kim-kv/core/page_handle.h"
#include "kim-kv/core/page_state.h"

#include <cstdint>
#include <vector>

namespace kimkvcache {

class FixedPageManager;
class KvCacheManager;

struct MappingEntry final {
    std::uint32_t logical_token_begin{0};
    std::uint16_t valid_tokens{0};
    PageKind kind{PageKind::Micro};
    PageHandle handle{PageHandle::invalid()};

    [[nodiscard]] constexpr std::uint32_t logicalTokenEnd() const noexcept
    {
        return logical_token_begin + valid_tokens;
    }

    friend constexpr bool operator==(MappingEntry const& a, MappingEntry const& b) noexcept
    {
        return a.logical_token_begin == b.logical_token_begin && a.valid_tokens == b.valid_tokens
            && a.kind == b.kind && a.handle == b.handle;
    }
    friend constexpr bool operator!=(MappingEntry const& a, MappingEntry const& b) noexcept { return !(a == b); }
};

class BlockTable final {
public:
    BlockTable() = default;

    [[nodiscard]] std::uint64_t version() const noexcept { return version_; }
    [[nodiscard]] std::uint32_t tokenCount() const noexcept
    {
        return entries_.empty() ? 0 : entries_.back().logicalTokenEnd();
    }
    [[nodiscard]] bool empty() const noexcept { return entries_.empty(); }
    [[nodiscard]] std::vector<MappingEntry> const& entries() const noexcept { return entries_; }

    // Entry covering `logical_token`, or nullptr.
    [[nodiscard]] MappingEntry const* find(std::uint32_t logical_token) const noexcept;

    // Contiguous from 0, valid handles of the entry's kind, 1..capacity tokens
    // each (standard capacities), no physical page mapped twice.
    [[nodiscard]] bool checkInvariants() const;
    // Same with one uniform page capacity (fixed-size page tables).
    [[nodiscard]] bool checkInvariants(std::uint16_t uniform_page_token_capacity) const;

private:
    friend class KvCacheManager;
    friend class FixedPageManager;

    std::vector<MappingEntry> entries_;
    std::uint64_t version_{0};
};

}  // namespace kimkvcache
