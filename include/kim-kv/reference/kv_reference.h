// CPU reference surface of the reference's public API
// (include/kim-kv/reference/kv_reference.h:10-23): the binary16 codec used for
// every KV element and a contiguous-layout attention comparator.  Host code
// only: no HIP path calls these; they exist so that callers of the
// reference's "stable CPU API" compile and behave the same against this
// library.
#pragma once

#include "kim-kv/core/kv_layout.h"

#include <cstdint>
#include <vector>

namespace kimkvcache {

// float -> IEEE binary16 bits, round to nearest even (subnormals, +-0,
// overflow to infinity, NaN kept NaN).
[[nodiscard]] KvScalar floatToKvScalar(float value) noexcept;

// IEEE binary16 bits -> float (exact).
[[nodiscard]] float kvScalarToFloat(KvScalar value) noexcept;

// Multi-head attention of one query per (layer, head) over a contiguous
// history: kv [layer][K/V][token][head][dim] (token_count tokens), query and
// output [layer][head][dim] fp32; s_t = (q . k_t) / sqrt(head_dim), softmax
// with the maximum subtracted, fp32 accumulation.  false (output untouched)
// for an invalid layout, zero tokens or mismatched sizes.
[[nodiscard]] bool referenceAttention(KvLayout const& layout, std::vector<KvScalar> const& contiguous_kv,
                                      std::uint32_t token_count, std::vector<float> const& query,
                                      std::vector<float>& output);

}  // namespace kimkvcache
