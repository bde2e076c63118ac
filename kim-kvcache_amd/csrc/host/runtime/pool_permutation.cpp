#include "kim-kv/runtime/pool_permutation.h"

#include <utility>
#include <vector>

namespace kimkvcache {
namespace {

std::uint64_t splitmixNext(std::uint64_t& state)
{
    state += 0x9E3779B97F4A7C15ull;
    std::uint64_t z = state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

}  // namespace

void seededPermutation(std::uint64_t seed, std::uint32_t n, std::uint32_t* out)
{
    for (std::uint32_t i = 0; i < n; ++i) out[i] = i;
    std::uint64_t state = seed;
    for (std::uint32_t i = n; i > 1; --i) {
        std::uint32_t const j = static_cast<std::uint32_t>(splitmixNext(state) % i);
        std::swap(out[i - 1], out[j]);
    }
}

KvCacheError permuteFreeSlotsOf(KvCacheManager& mgr, PageKind kind, std::uint64_t seed)
{
    KvCacheManagerSnapshot const snap = mgr.snapshot();
    PagePoolSnapshot const pool = kind == PageKind::Micro ? snap.micro_pool : snap.extent_pool;
    std::uint32_t const n = pool.total_slots;
    if (pool.free_slots != n) return KvCacheError::InvalidState;
    std::vector<std::uint32_t> perm(n);
    seededPermutation(seed, n, perm.data());
    constexpr std::uint64_t kBase = 0xFFFF000000000000ull;
    std::vector<std::uint64_t> owner(n, 0);
    for (std::uint32_t i = 0; i < n; ++i) {
        std::uint64_t const id = kBase + i;
        KvCacheError e = mgr.createRequest(id);
        if (e != KvCacheError::None) return e;
        if (kind == PageKind::Micro) {
            e = mgr.append(id, kMicroPageTokenCapacity);
        } else {
            e = mgr.append(id, kExtentPageTokenCapacity);
            if (e == KvCacheError::None) {
                PromotionPrepareResult const p = mgr.preparePromotion(id, 0);
                e = p.error;
                if (e == KvCacheError::None) e = mgr.commitPromotion(p.promotion_id);
            }
        }
        if (e != KvCacheError::None) return e;
        std::optional<BlockTable> t = mgr.blockTable(id);
        if (!t.has_value() || t->entries().size() != 1) return KvCacheError::InternalInvariantViolation;
        owner[t->entries()[0].handle.slot] = id;
    }
    for (std::uint32_t k = n; k > 0; --k) {
        KvCacheError const e = mgr.releaseRequest(owner[perm[k - 1]]);
        if (e != KvCacheError::None) return e;
    }
    return KvCacheError::None;
}

}  // namespace kimkvcache
