// Seeded scattering of a pool's free list (benchmark and test workloads whose
// page ids must be a random permutation of the pool; no reference
// counterpart).  Uses only the public manager API, so the manager's state
// afterwards is exactly what an allocator-driven workload would produce.
#pragma once

#include "kim-kv/core/page_types.h"
#include "kim-kv/runtime/kv_cache_manager.h"

#include <cstdint>

namespace kimkvcache {

// Fisher-Yates over [0, n) driven by splitmix64(seed): out[i] is the i-th
// element of the permutation.
void seededPermutation(std::uint64_t seed, std::uint32_t n, std::uint32_t* out);

// With every slot of `kind` free, allocates all of them through throw-away
// requests (ids 0xFFFF000000000000 + i) and releases them in reverse
// permutation order, so the LIFO free list hands out perm[0], perm[1], ...
// Returns InvalidState when a slot of that pool is in use.
[[nodiscard]] KvCacheError permuteFreeSlotsOf(KvCacheManager& manager, PageKind kind, std::uint64_t seed);

}  // namespace kimkvcache
