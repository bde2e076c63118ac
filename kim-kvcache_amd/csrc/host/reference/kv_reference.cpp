// CPU reference surface (include/kim-kv/reference/kv_reference.h): the
// binary16 codec and the contiguous attention comparator of the reference's
// public API (src/reference/kv_reference.cpp:31-234 defines the behaviour:
// round-to-nearest-even encode with subnormals, exact decode, scale applied
// after the dot product, max-subtracted softmax in fp32).  Written from the
// IEEE-754 binary16 format: 1 sign bit, 5 exponent bits (bias 15), 10
// fraction bits; subnormals are fraction * 2^-24.
#include "kim-kv/reference/kv_reference.h"

#include <cmath>
#include <cstring>
#include <limits>
#include <utility>

namespace kimkvcache {
namespace {

std::uint32_t bitsOf(float v) noexcept
{
    std::uint32_t b = 0;
    std::memcpy(&b, &v, sizeof(b));
    return b;
}

float floatOf(std::uint32_t b) noexcept
{
    float v = 0.0F;
    std::memcpy(&v, &b, sizeof(v));
    return v;
}

// q = x >> shift rounded to nearest, ties to even (1 <= shift <= 31).
std::uint32_t shiftRoundEven(std::uint32_t x, std::uint32_t shift) noexcept
{
    std::uint32_t const q = x >> shift;
    std::uint32_t const rest = x & ((1u << shift) - 1u);
    std::uint32_t const half = 1u << (shift - 1u);
    return q + ((rest > half || (rest == half && (q & 1u) != 0)) ? 1u : 0u);
}

}  // namespace

KvScalar floatToKvScalar(float value) noexcept
{
    std::uint32_t const bits = bitsOf(value);
    auto const sign = static_cast<std::uint16_t>((bits >> 16) & 0x8000u);
    std::uint32_t const magnitude = bits & 0x7FFFFFFFu;
    std::uint32_t const exponent = magnitude >> 23;      // fp32 biased exponent
    if (exponent == 0xFFu) {                              // infinity or NaN (quiet)
        return static_cast<KvScalar>(sign | ((magnitude & 0x7FFFFFu) != 0 ? 0x7E00u : 0x7C00u));
    }
    // 65520 = 65504 + half an ulp rounds (to even) to infinity.
    if (magnitude >= 0x477FF000u) return static_cast<KvScalar>(sign | 0x7C00u);
    if (exponent >= 113) {                                // >= 2^-14: a normal binary16
        // Rebias 127 -> 15 and drop 13 fraction bits; a carry out of the
        // fraction moves into the exponent, which is the correct result.
        std::uint32_t const rebased = magnitude - (112u << 23);
        return static_cast<KvScalar>(sign | shiftRoundEven(rebased, 13));
    }
    if (exponent < 102) return sign;                      // below 2^-25: rounds to zero
    // Subnormal: value / 2^-24 = significand * 2^(exponent - 126).
    std::uint32_t const significand = (magnitude & 0x7FFFFFu) | 0x800000u;
    return static_cast<KvScalar>(sign | shiftRoundEven(significand, 126u - exponent));
}

float kvScalarToFloat(KvScalar value) noexcept
{
    std::uint32_t const sign = (static_cast<std::uint32_t>(value) & 0x8000u) << 16;
    std::uint32_t const exponent = (value >> 10) & 0x1Fu;
    std::uint32_t const fraction = value & 0x3FFu;
    if (exponent == 0x1Fu) return floatOf(sign | 0x7F800000u | (fraction << 13));
    if (exponent == 0) {
        float const magnitude = std::ldexp(static_cast<float>(fraction), -24);
        return sign != 0 ? -magnitude : magnitude;
    }
    return floatOf(sign | ((exponent + 112u) << 23) | (fraction << 13));
}

bool referenceAttention(KvLayout const& layout, std::vector<KvScalar> const& kv, std::uint32_t token_count,
                        std::vector<float> const& query, std::vector<float>& output)
{
    std::size_t kv_elements = 0;
    if (!layout.valid() || token_count == 0 || !layout.elementsForTokens(token_count, kv_elements)
        || kv.size() != kv_elements) {
        return false;
    }
    std::size_t const rows = static_cast<std::size_t>(layout.layer_count) * layout.kv_head_count;
    std::size_t const D = layout.head_dimension;
    if (query.size() != rows * D) return false;

    std::vector<float> result(rows * D, 0.0F);
    std::vector<float> score(token_count);
    float const scale = 1.0F / std::sqrt(static_cast<float>(D));
    for (std::uint32_t l = 0; l < layout.layer_count; ++l) {
        for (std::uint32_t h = 0; h < layout.kv_head_count; ++h) {
            float const* q = query.data() + (static_cast<std::size_t>(l) * layout.kv_head_count + h) * D;
            float best = -std::numeric_limits<float>::infinity();
            for (std::uint32_t t = 0; t < token_count; ++t) {
                std::size_t const k0 = layout.offset(l, KvComponent::Key, t, h, 0, token_count);
                float dot = 0.0F;
                for (std::size_t d = 0; d < D; ++d) dot += q[d] * kvScalarToFloat(kv[k0 + d]);
                score[t] = dot * scale;
                best = std::fmax(best, score[t]);
            }
            float* o = result.data() + (static_cast<std::size_t>(l) * layout.kv_head_count + h) * D;
            float denominator = 0.0F;
            for (std::uint32_t t = 0; t < token_count; ++t) {
                float const w = std::exp(score[t] - best);
                denominator += w;
                std::size_t const v0 = layout.offset(l, KvComponent::Value, t, h, 0, token_count);
                for (std::size_t d = 0; d < D; ++d) o[d] += w * kvScalarToFloat(kv[v0 + d]);
            }
            for (std::size_t d = 0; d < D; ++d) o[d] /= denominator;
        }
    }
    output = std::move(result);
    return true;
}

}  // namespace kimkvcache
