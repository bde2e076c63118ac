// C facade over KvCacheManager (include/kimkv_host.h, kimkv_manager_*).
#include "kimkv_host.h"

#include "capi_internal.h"
#include "kim-kv/runtime/kv_cache_manager.h"
#include "kim-kv/runtime/pool_permutation.h"

#include <new>
#include <optional>
#include <vector>

using namespace kimkvcache;

namespace {

int code(KvCacheError e) { return static_cast<int>(e); }

PageHandle toHandle(kimkv_page_handle h) { return PageHandle{static_cast<PageKind>(h.kind), h.slot, h.generation}; }

kimkv_page_handle fromHandle(PageHandle h)
{
    return kimkv_page_handle{static_cast<std::uint32_t>(h.kind), h.slot, h.generation};
}

int copyTable(BlockTable const& t, std::uint64_t* version, kimkv_mapping_entry* out, std::uint32_t capacity,
              std::uint32_t* count)
{
    auto const& e = t.entries();
    if (version) *version = t.version();
    if (count) *count = static_cast<std::uint32_t>(e.size());
    if (out == nullptr) return 0;
    if (e.size() > capacity) return code(KvCacheError::InvalidArgument);
    for (std::size_t i = 0; i < e.size(); ++i) {
        out[i] = kimkv_mapping_entry{e[i].logical_token_begin, e[i].valid_tokens, static_cast<std::uint8_t>(e[i].kind),
                                     0, e[i].handle.slot, e[i].handle.generation};
    }
    return 0;
}

void poolOut(PagePoolSnapshot const& p, kimkv_pool_snapshot* o)
{
    *o = kimkv_pool_snapshot{static_cast<std::uint32_t>(p.kind), p.total_slots, p.free_slots, p.allocated_slots,
                             p.successful_allocations, p.successful_releases, p.failed_allocations,
                             p.rejected_releases};
}

}  // namespace

extern "C" {

kimkv_manager* kimkv_manager_create(uint32_t micro_capacity, uint32_t extent_capacity)
{
    try {
        auto owned = std::make_unique<KvCacheManager>(micro_capacity, extent_capacity);
        KvCacheManager* raw = owned.get();
        return new kimkv_manager{std::move(owned), raw};
    } catch (...) {
        return nullptr;
    }
}

void kimkv_manager_destroy(kimkv_manager* m) { delete m; }

int kimkv_manager_create_request(kimkv_manager* m, uint64_t id) { return code(m->m->createRequest(id)); }
int kimkv_manager_append(kimkv_manager* m, uint64_t id, uint32_t n) { return code(m->m->append(id, n)); }

int kimkv_manager_reserve_token(kimkv_manager* m, uint64_t id, uint32_t expected, uint64_t* reservation_id,
                                uint64_t* reserved_version, kimkv_mapping_entry* entries, uint32_t capacity,
                                uint32_t* count)
{
    TokenReservationResult r = m->m->reserveToken(id, expected);
    if (reservation_id) *reservation_id = r.reservation_id;
    if (r.error != KvCacheError::None) {
        if (count) *count = 0;
        return code(r.error);
    }
    return copyTable(r.reserved, reserved_version, entries, capacity, count);
}

int kimkv_manager_commit_token(kimkv_manager* m, uint64_t r) { return code(m->m->commitTokenReservation(r)); }
int kimkv_manager_rollback_token(kimkv_manager* m, uint64_t r) { return code(m->m->rollbackTokenReservation(r)); }
int kimkv_manager_seal_tail(kimkv_manager* m, uint64_t id) { return code(m->m->sealTail(id)); }
int kimkv_manager_fork_request(kimkv_manager* m, uint64_t s, uint64_t c) { return code(m->m->forkRequest(s, c)); }
int kimkv_manager_release_request(kimkv_manager* m, uint64_t id) { return code(m->m->releaseRequest(id)); }

int kimkv_manager_prepare_promotion(kimkv_manager* m, uint64_t id, uint32_t begin, uint64_t* promotion_id,
                                    kimkv_page_handle* sources, kimkv_page_handle* target)
{
    PromotionPrepareResult r = m->m->preparePromotion(id, begin);
    if (promotion_id) *promotion_id = r.promotion_id;
    if (sources) {
        for (std::size_t i = 0; i < kPromotionSourcePageCount; ++i) sources[i] = fromHandle(r.source_handles[i]);
    }
    if (target) *target = fromHandle(r.target_handle);
    return code(r.error);
}

int kimkv_manager_commit_promotion(kimkv_manager* m, uint64_t p) { return code(m->m->commitPromotion(p)); }
int kimkv_manager_rollback_promotion(kimkv_manager* m, uint64_t p) { return code(m->m->rollbackPromotion(p)); }

int kimkv_manager_acquire_request_lease(kimkv_manager* m, uint64_t id, uint64_t* lease)
{
    PageLeaseAcquireResult r = m->m->acquireRequestReadLease(id);
    if (lease) *lease = r.lease_id;
    return code(r.error);
}

int kimkv_manager_acquire_promotion_lease(kimkv_manager* m, uint64_t p, uint64_t* lease)
{
    PageLeaseAcquireResult r = m->m->acquirePromotionIoLease(p);
    if (lease) *lease = r.lease_id;
    return code(r.error);
}

int kimkv_manager_acquire_reservation_lease(kimkv_manager* m, uint64_t r, uint64_t* lease)
{
    PageLeaseAcquireResult res = m->m->acquireTokenReservationLease(r);
    if (lease) *lease = res.lease_id;
    return code(res.error);
}

int kimkv_manager_release_lease(kimkv_manager* m, uint64_t lease) { return code(m->m->releasePageLease(lease)); }

int kimkv_manager_block_table(const kimkv_manager* m, uint64_t id, uint64_t* version, kimkv_mapping_entry* entries,
                              uint32_t capacity, uint32_t* count)
{
    std::optional<BlockTable> t = m->m->blockTable(id);
    if (!t.has_value()) {
        if (count) *count = 0;
        return code(KvCacheError::RequestNotFound);
    }
    return copyTable(*t, version, entries, capacity, count);
}

int kimkv_manager_page_metadata(const kimkv_manager* m, kimkv_page_handle h, kimkv_page_metadata* out)
{
    std::optional<PageMetadataSnapshot> s = m->m->pageMetadata(toHandle(h));
    if (!s.has_value()) return 1;
    *out = kimkv_page_metadata{static_cast<std::uint32_t>(s->state), s->valid_tokens, s->ref_count,
                               s->promotion_pins, s->inflight_readers, 0, s->mutable_owner};
    return 0;
}

void kimkv_manager_get_snapshot(const kimkv_manager* m, kimkv_manager_snapshot* out)
{
    KvCacheManagerSnapshot const s = m->m->snapshot();
    out->request_count = s.request_count;
    out->promotion_count = s.promotion_count;
    out->page_lease_count = s.page_lease_count;
    out->token_reservation_count = s.token_reservation_count;
    poolOut(s.micro_pool, &out->micro_pool);
    poolOut(s.extent_pool, &out->extent_pool);
}

int kimkv_manager_check_invariants(const kimkv_manager* m) { return m->m->checkInvariants() ? 1 : 0; }

void kimkv_seeded_permutation(uint64_t seed, uint32_t n, uint32_t* out) { seededPermutation(seed, n, out); }

int kimkv_manager_permute_free_slots(kimkv_manager* m, uint32_t kind, uint64_t seed)
{
    if (kind > 1) return code(KvCacheError::InvalidState);
    return code(permuteFreeSlotsOf(*m->m, kind == 0 ? PageKind::Micro : PageKind::Extent, seed));
}

}  // extern "C"
