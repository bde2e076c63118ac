// ref_driver.cpp -- TEST INFRASTRUCTURE ONLY.
//
// C entry points over the reference's own CPU library (src/core, src/runtime,
// src/reference under the reference tree), compiled by oracle/build.py into
// oracle/_ref/libkimkv_ref.so.  The functions mirror include/kimkv_host.h's
// kimkv_manager_* facade with a kvref_ prefix, so tests can run one operation
// trace against the reference and against libkimkv.so and compare page tables,
// page metadata and error codes bit for bit.  Nothing here is shipped.
#include "kim-kv/reference/kv_reference.h"
#include "kim-kv/runtime/kv_cache_manager.h"

#include "kimkv_host.h"

#include <cstdint>
#include <cstring>
#include <new>
#include <optional>
#include <unordered_map>
#include <vector>

using namespace kimkvcache;

namespace {

int code(KvCacheError e) { return static_cast<int>(e); }

PageHandle to_handle(kimkv_page_handle h)
{
    return PageHandle{static_cast<PageKind>(h.kind), h.slot, h.generation};
}

kimkv_page_handle from_handle(PageHandle h)
{
    return kimkv_page_handle{static_cast<uint32_t>(h.kind), h.slot, h.generation};
}

int copy_table(BlockTable const& table, uint64_t* version, kimkv_mapping_entry* entries, uint32_t capacity,
               uint32_t* count)
{
    auto const& e = table.entries();
    if (version) *version = table.version();
    if (count) *count = static_cast<uint32_t>(e.size());
    if (entries == nullptr) return 0;
    if (e.size() > capacity) return code(KvCacheError::InvalidArgument);
    for (size_t i = 0; i < e.size(); ++i) {
        entries[i] = kimkv_mapping_entry{e[i].logical_token_begin, e[i].valid_tokens,
                                         static_cast<uint8_t>(e[i].kind), 0, e[i].handle.slot,
                                         e[i].handle.generation};
    }
    return 0;
}

uint64_t splitmix_next(uint64_t& state)
{
    state += 0x9E3779B97F4A7C15ull;
    uint64_t z = state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void permutation(uint64_t seed, uint32_t n, uint32_t* out)
{
    for (uint32_t i = 0; i < n; ++i) out[i] = i;
    uint64_t state = seed;
    for (uint32_t i = n; i > 1; --i) {
        uint32_t const j = static_cast<uint32_t>(splitmix_next(state) % i);
        uint32_t const tmp = out[i - 1];
        out[i - 1] = out[j];
        out[j] = tmp;
    }
}

}  // namespace

struct kvref_manager {
    KvCacheManager m;
    kvref_manager(uint32_t micro, uint32_t extent) : m(micro, extent) {}
};

extern "C" {

kvref_manager* kvref_manager_create(uint32_t micro_capacity, uint32_t extent_capacity)
{
    try {
        return new kvref_manager(micro_capacity, extent_capacity);
    } catch (...) {
        return nullptr;
    }
}

void kvref_manager_destroy(kvref_manager* m) { delete m; }

int kvref_manager_create_request(kvref_manager* m, uint64_t id) { return code(m->m.createRequest(id)); }

int kvref_manager_append(kvref_manager* m, uint64_t id, uint32_t n) { return code(m->m.append(id, n)); }

int kvref_manager_reserve_token(kvref_manager* m, uint64_t id, uint32_t expected, uint64_t* reservation_id,
                                uint64_t* reserved_version, kimkv_mapping_entry* entries, uint32_t capacity,
                                uint32_t* count)
{
    TokenReservationResult r = m->m.reserveToken(id, expected);
    if (reservation_id) *reservation_id = r.reservation_id;
    if (r.error != KvCacheError::None) {
        if (count) *count = 0;
        return code(r.error);
    }
    int const rc = copy_table(r.reserved, reserved_version, entries, capacity, count);
    return rc;
}

int kvref_manager_commit_token(kvref_manager* m, uint64_t r) { return code(m->m.commitTokenReservation(r)); }
int kvref_manager_rollback_token(kvref_manager* m, uint64_t r) { return code(m->m.rollbackTokenReservation(r)); }
int kvref_manager_seal_tail(kvref_manager* m, uint64_t id) { return code(m->m.sealTail(id)); }
int kvref_manager_fork_request(kvref_manager* m, uint64_t s, uint64_t c) { return code(m->m.forkRequest(s, c)); }
int kvref_manager_release_request(kvref_manager* m, uint64_t id) { return code(m->m.releaseRequest(id)); }

int kvref_manager_prepare_promotion(kvref_manager* m, uint64_t id, uint32_t begin, uint64_t* promotion_id,
                                    kimkv_page_handle* sources, kimkv_page_handle* target)
{
    PromotionPrepareResult r = m->m.preparePromotion(id, begin);
    if (promotion_id) *promotion_id = r.promotion_id;
    if (sources) {
        for (size_t i = 0; i < kPromotionSourcePageCount; ++i) sources[i] = from_handle(r.source_handles[i]);
    }
    if (target) *target = from_handle(r.target_handle);
    return code(r.error);
}

int kvref_manager_commit_promotion(kvref_manager* m, uint64_t p) { return code(m->m.commitPromotion(p)); }
int kvref_manager_rollback_promotion(kvref_manager* m, uint64_t p) { return code(m->m.rollbackPromotion(p)); }

int kvref_manager_acquire_request_lease(kvref_manager* m, uint64_t id, uint64_t* lease)
{
    PageLeaseAcquireResult r = m->m.acquireRequestReadLease(id);
    if (lease) *lease = r.lease_id;
    return code(r.error);
}

int kvref_manager_acquire_promotion_lease(kvref_manager* m, uint64_t p, uint64_t* lease)
{
    PageLeaseAcquireResult r = m->m.acquirePromotionIoLease(p);
    if (lease) *lease = r.lease_id;
    return code(r.error);
}

int kvref_manager_acquire_reservation_lease(kvref_manager* m, uint64_t r, uint64_t* lease)
{
    PageLeaseAcquireResult res = m->m.acquireTokenReservationLease(r);
    if (lease) *lease = res.lease_id;
    return code(res.error);
}

int kvref_manager_release_lease(kvref_manager* m, uint64_t lease) { return code(m->m.releasePageLease(lease)); }

int kvref_manager_block_table(const kvref_manager* m, uint64_t id, uint64_t* version, kimkv_mapping_entry* entries,
                              uint32_t capacity, uint32_t* count)
{
    std::optional<BlockTable> t = m->m.blockTable(id);
    if (!t.has_value()) {
        if (count) *count = 0;
        return code(KvCacheError::RequestNotFound);
    }
    return copy_table(*t, version, entries, capacity, count);
}

int kvref_manager_page_metadata(const kvref_manager* m, kimkv_page_handle h, kimkv_page_metadata* out)
{
    std::optional<PageMetadataSnapshot> s = m->m.pageMetadata(to_handle(h));
    if (!s.has_value()) return 1;
    out->state = static_cast<uint32_t>(s->state);
    out->valid_tokens = s->valid_tokens;
    out->ref_count = s->ref_count;
    out->promotion_pins = s->promotion_pins;
    out->inflight_readers = s->inflight_readers;
    out->reserved = 0;
    out->mutable_owner = s->mutable_owner;
    return 0;
}

static void pool_out(PagePoolSnapshot const& p, kimkv_pool_snapshot* o)
{
    o->kind = static_cast<uint32_t>(p.kind);
    o->total_slots = p.total_slots;
    o->free_slots = p.free_slots;
    o->allocated_slots = p.allocated_slots;
    o->successful_allocations = p.successful_allocations;
    o->successful_releases = p.successful_releases;
    o->failed_allocations = p.failed_allocations;
    o->rejected_releases = p.rejected_releases;
}

void kvref_manager_get_snapshot(const kvref_manager* m, kimkv_manager_snapshot* out)
{
    KvCacheManagerSnapshot const s = m->m.snapshot();
    out->request_count = s.request_count;
    out->promotion_count = s.promotion_count;
    out->page_lease_count = s.page_lease_count;
    out->token_reservation_count = s.token_reservation_count;
    pool_out(s.micro_pool, &out->micro_pool);
    pool_out(s.extent_pool, &out->extent_pool);
}

int kvref_manager_check_invariants(const kvref_manager* m) { return m->m.checkInvariants() ? 1 : 0; }

void kvref_seeded_permutation(uint64_t seed, uint32_t n, uint32_t* out) { permutation(seed, n, out); }

// Same public-API call sequence as kimkv_manager_permute_free_slots.
int kvref_manager_permute_free_slots(kvref_manager* m, uint32_t kind, uint64_t seed)
{
    KvCacheManager& mgr = m->m;
    KvCacheManagerSnapshot const snap = mgr.snapshot();
    PagePoolSnapshot const pool = kind == 0 ? snap.micro_pool : snap.extent_pool;
    uint32_t const n = pool.total_slots;
    if (pool.free_slots != n || kind > 1) return code(KvCacheError::InvalidState);
    std::vector<uint32_t> perm(n);
    permutation(seed, n, perm.data());
    constexpr uint64_t kBase = 0xFFFF000000000000ull;
    std::vector<uint64_t> owner(n, 0);
    for (uint32_t i = 0; i < n; ++i) {
        uint64_t const id = kBase + i;
        KvCacheError e = mgr.createRequest(id);
        if (e != KvCacheError::None) return code(e);
        if (kind == 0) {
            e = mgr.append(id, kMicroPageTokenCapacity);
        } else {
            e = mgr.append(id, kExtentPageTokenCapacity);
            if (e == KvCacheError::None) {
                PromotionPrepareResult const p = mgr.preparePromotion(id, 0);
                e = p.error;
                if (e == KvCacheError::None) e = mgr.commitPromotion(p.promotion_id);
            }
        }
        if (e != KvCacheError::None) return code(e);
        std::optional<BlockTable> t = mgr.blockTable(id);
        if (!t.has_value() || t->entries().size() != 1) return code(KvCacheError::InternalInvariantViolation);
        owner[t->entries()[0].handle.slot] = id;
    }
    for (uint32_t k = n; k > 0; --k) {
        KvCacheError const e = mgr.releaseRequest(owner[perm[k - 1]]);
        if (e != KvCacheError::None) return code(e);
    }
    return 0;
}

uint16_t kvref_float_to_kv(float v) { return floatToKvScalar(v); }
float kvref_kv_to_float(uint16_t v) { return kvScalarToFloat(v); }

int kvref_reference_attention(uint32_t layers, uint32_t heads, uint32_t dim, const uint16_t* kv,
                              uint32_t token_count, const float* query, float* output)
{
    KvLayout const layout{layers, heads, dim};
    size_t elements = 0;
    if (!layout.elementsForTokens(token_count, elements)) return 0;
    std::vector<KvScalar> kvv(kv, kv + elements);
    std::vector<float> q(query, query + static_cast<size_t>(layers) * heads * dim);
    std::vector<float> out;
    if (!referenceAttention(layout, kvv, token_count, q, out)) return 0;
    std::memcpy(output, out.data(), out.size() * sizeof(float));
    return 1;
}

}  // extern "C"
