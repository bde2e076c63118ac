// KV tensor layout (include/kim-kv/core/kv_layout.h of the reference).  The
// contiguous order [layer][K/V][token][head][dim] is the one append inputs and
// gather outputs use; device pages use their own private layout.
#pragma once

#include "kim-kv/core/page_state.h"

#include <cstddef>
#include <cstdint>
#include <limits>

namespace kimkvcache {

using KvScalar = std::uint16_t;   // raw IEEE binary16 bits

enum class KvComponent : std::uint8_t {
    Key = 0,
    Value = 1,
};

struct KvLayout final {
    std::uint32_t layer_count{0};
    std::uint32_t kv_head_count{0};
    std::uint32_t head_dimension{0};

    [[nodiscard]] constexpr bool valid() const noexcept
    {
        return layer_count != 0 && kv_head_count != 0 && head_dimension != 0;
    }

    [[nodiscard]] bool elementsPerToken(std::size_t& result) const noexcept
    {
        if (!valid()) return false;
        std::size_t v = layer_count;
        if (!mul(v, 2, v) || !mul(v, kv_head_count, v) || !mul(v, head_dimension, v)) return false;
        result = v;
        return true;
    }

    [[nodiscard]] bool elementsForTokens(std::uint32_t tokens, std::size_t& result) const noexcept
    {
        std::size_t per = 0;
        return elementsPerToken(per) && mul(per, tokens, result);
    }

    [[nodiscard]] bool bytesForTokens(std::uint32_t tokens, std::size_t& result) const noexcept
    {
        std::size_t e = 0;
        return elementsForTokens(tokens, e) && mul(e, sizeof(KvScalar), result);
    }

    [[nodiscard]] bool pageElements(PageKind kind, std::size_t& result) const noexcept
    {
        return elementsForTokens(pageTokenCapacity(kind), result);
    }

    // [layer][K/V][token][head][dim] within a buffer of `token_capacity` tokens.
    [[nodiscard]] std::size_t offset(std::uint32_t layer, KvComponent component, std::uint32_t token,
                                     std::uint32_t head, std::uint32_t dimension,
                                     std::uint32_t token_capacity) const noexcept
    {
        return (((static_cast<std::size_t>(layer) * 2 + static_cast<std::uint8_t>(component)) * token_capacity
                 + token) * kv_head_count + head) * head_dimension + dimension;
    }

private:
    [[nodiscard]] static bool mul(std::size_t a, std::size_t b, std::size_t& out) noexcept
    {
        if (a != 0 && b > std::numeric_limits<std::size_t>::max() / a) return false;
        out = a * b;
        return true;
    }
};

}  // namespace kimkvcache
