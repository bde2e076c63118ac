// BlockTable lookup and structural invariants (semantics of
// src/core/block_table.cpp:12-130 in the reference).
#include "kim-kv/core/block_table.h"

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <limits>
#include <vector>

namespace kimkvcache {
namespace {

// True when no physical page appears twice.  Pairwise for short tables; for
// long ones an open-addressing set on (kind, slot) with per-call stamps (no
// clearing), comparing the generation on a (kind, slot) hit: same answer as
// comparing every pair, linear time.
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
    struct Slot {
        std::uint64_t key;
        std::uint32_t generation;
        std::uint32_t stamp;
    };
    thread_local std::vector<Slot> set;
    thread_local std::uint32_t stamp = 0;
    std::size_t cap = 64;
    while (cap < 2 * n) cap <<= 1;
    if (set.size() < cap) set.assign(cap, Slot{0, 0, 0});
    if (++stamp == 0) {
        for (Slot& s : set) s.stamp = 0;
        stamp = 1;
    }
    std::size_t const mask = cap - 1;
    for (MappingEntry const& e : entries) {
        std::uint64_t const key = (static_cast<std::uint64_t>(e.handle.kind) << 32) | e.handle.slot;
        std::size_t h = static_cast<std::size_t>((key * 0x9E3779B97F4A7C15ull) >> 32) & mask;
        while (set[h].stamp == stamp) {
            if (set[h].key == key && set[h].generation == e.handle.generation) return false;
            h = (h + 1) & mask;
        }
        set[h] = Slot{key, e.handle.generation, stamp};
    }
    return true;
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
