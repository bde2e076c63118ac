// BlockTable lookup and structural invariants (semantics of
// src/core/block_table.cpp:12-130 in the reference).
#include "kim-kv/core/block_table.h"

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <limits>
#include <tuple>
#include <vector>

namespace kimkvcache {
namespace {

// True when no physical page appears twice.  Pairwise for short tables, a
// sort of the handles for long ones (same answer, O(n log n)).
bool handlesDistinct(std::vector<MappingEntry> const& entries)
{
    std::size_t const n = entries.size();
    if (n <= 32) {
        for (std::size_t i = 1; i < n; ++i) {
            for (std::size_t j = 0; j < i; ++j) {
                if (entries[i].handle == entries[j].handle) return false;
            }
        }
        return true;
    }
    std::vector<std::tuple<std::uint8_t, std::uint32_t, std::uint32_t>> keys;
    keys.reserve(n);
    for (MappingEntry const& e : entries) {
        keys.emplace_back(static_cast<std::uint8_t>(e.handle.kind), e.handle.slot, e.handle.generation);
    }
    std::sort(keys.begin(), keys.end());
    return std::adjacent_find(keys.begin(), keys.end()) == keys.end();
}

bool tableValid(std::vector<MappingEntry> const& entries, std::uint16_t uniform_capacity)
{
    std::uint64_t next = 0;
    for (MappingEntry const& e : entries) {
        if (!e.handle.isStructurallyValid() || e.kind != e.handle.kind) return false;
        std::uint16_t const cap = uniform_capacity == 0 ? pageTokenCapacity(e.kind) : uniform_capacity;
        if (cap == 0 || e.valid_tokens == 0 || e.valid_tokens > cap) return false;
        if (next > std::numeric_limits<std::uint32_t>::max() || e.logical_token_begin != next) return false;
        next += e.valid_tokens;
        if (next > std::numeric_limits<std::uint32_t>::max()) return false;
    }
    return handlesDistinct(entries);
}

}  // namespace

MappingEntry const* BlockTable::find(std::uint32_t logical_token) const noexcept
{
    auto const upper = std::upper_bound(
        entries_.begin(), entries_.end(), logical_token,
        [](std::uint32_t token, MappingEntry const& e) { return token < e.logical_token_begin; });
    if (upper == entries_.begin()) return nullptr;
    MappingEntry const& candidate = *(upper - 1);
    return logical_token < candidate.logicalTokenEnd() ? &candidate : nullptr;
}

bool BlockTable::checkInvariants() const { return tableValid(entries_, 0); }

bool BlockTable::checkInvariants(std::uint16_t uniform_page_token_capacity) const
{
    return uniform_page_token_capacity != 0 && tableValid(entries_, uniform_page_token_capacity);
}

}  // namespace kimkvcache
