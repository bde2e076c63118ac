// PageHandle: (kind, slot, generation) (include/kim-kv/core/page_handle.h of the reference).
#pragma once

#include "kim-kv/core/page_types.h"

#include <cstdint>
#include <limits>
#include <type_traits>

namespace kimkvcache {

struct PageHandle final {
    static constexpr std::uint32_t kInvalidSlot = std::numeric_limits<std::uint32_t>::max();
    static constexpr std::uint32_t kInvalidGeneration = 0;

    PageKind kind{PageKind::Micro};
    std::uint32_t slot{kInvalidSlot};
    std::uint32_t generation{kInvalidGeneration};

    [[nodiscard]] static constexpr PageHandle invalid() noexcept { return {}; }

    // Checks the encoding only; the pool decides liveness.
    [[nodiscard]] constexpr bool isStructurallyValid() const noexcept
    {
        return isKnownPageKind(kind) && slot != kInvalidSlot && generation != kInvalidGeneration;
    }

    friend constexpr bool operator==(PageHandle a, PageHandle b) noexcept
    {
        return a.kind == b.kind && a.slot == b.slot && a.generation == b.generation;
    }
    friend constexpr bool operator!=(PageHandle a, PageHandle b) noexcept { return !(a == b); }
};

static_assert(std::is_trivially_copyable_v<PageHandle>);
static_assert(std::is_standard_layout_v<PageHandle>);

}  // namespace kimkvcache
