// Twin-manager check of KvCacheManager's delta paths.  One manager is driven
// through the reference's calls (append, reserveToken), the other through
// appendWithLease / reserveTokenDelta, on the same seeded random operation
// sequences (create, append, reserve + commit or rollback, fork, seal,
// promotion, release) with small pools so that exhaustion is exercised.
// After every step both managers hold the same tables (entries and versions)
// and the same metadata for every page a table names, both pass their
// invariant checks, and each delta result describes exactly what changed.
#include "kim-kv/runtime/kv_cache_manager.h"

#include <cstdint>
#include <cstdio>
#include <optional>
#include <random>
#include <vector>

using namespace kimkvcache;

namespace {

int failures = 0;

#define CHECK(cond)                                                                  \
    do {                                                                             \
        if (!(cond)) {                                                               \
            std::printf("FAIL %s:%d: %s (seed %u step %d)\n", __FILE__, __LINE__, #cond, \
                        g_seed, g_step);                                             \
            ++failures;                                                              \
        }                                                                            \
    } while (0)

unsigned g_seed = 0;
int g_step = 0;

bool sameMetadata(std::optional<PageMetadataSnapshot> const& a, std::optional<PageMetadataSnapshot> const& b)
{
    if (a.has_value() != b.has_value()) return false;
    if (!a) return true;
    return a->state == b->state && a->valid_tokens == b->valid_tokens && a->ref_count == b->ref_count
        && a->promotion_pins == b->promotion_pins && a->inflight_readers == b->inflight_readers
        && a->mutable_owner == b->mutable_owner;
}

// Same table (or same absence) and the same metadata for every page it names.
void compareRequest(KvCacheManager const& a, KvCacheManager const& b, RequestId id)
{
    std::optional<BlockTable> const ta = a.blockTable(id);
    std::optional<BlockTable> const tb = b.blockTable(id);
    CHECK(ta.has_value() == tb.has_value());
    if (!ta || !tb) return;
    CHECK(ta->version() == tb->version());
    CHECK(ta->entries() == tb->entries());
    for (MappingEntry const& e : ta->entries()) CHECK(sameMetadata(a.pageMetadata(e.handle), b.pageMetadata(e.handle)));
}

void comparePools(KvCacheManager const& a, KvCacheManager const& b)
{
    KvCacheManagerSnapshot const sa = a.snapshot();
    KvCacheManagerSnapshot const sb = b.snapshot();
    CHECK(sa.request_count == sb.request_count);
    CHECK(sa.token_reservation_count == sb.token_reservation_count);
    CHECK(sa.page_lease_count == sb.page_lease_count);
    CHECK(sa.micro_pool.allocated_slots == sb.micro_pool.allocated_slots);
    CHECK(sa.extent_pool.allocated_slots == sb.extent_pool.allocated_slots);
    CHECK(a.checkInvariants());
    CHECK(b.checkInvariants());
}

void appendStep(KvCacheManager& a, KvCacheManager& b, RequestId id, std::uint32_t n)
{
    std::optional<BlockTable> const before = b.blockTable(id);
    KvCacheError const ea = a.append(id, n);
    AppendChange const c = b.appendWithLease(id, n);
    CHECK(ea == c.error);
    if (ea != KvCacheError::None) {
        CHECK(c.lease_id == kInvalidPageLeaseId);
        return;
    }
    CHECK(c.ok());
    std::optional<BlockTable> const after = b.blockTable(id);
    CHECK(before.has_value() && after.has_value());
    if (!before || !after) return;
    CHECK(c.logical_token_begin == before->tokenCount());
    CHECK(after->tokenCount() == before->tokenCount() + n);
    CHECK(c.version == after->version());
    CHECK(c.first_entry <= after->entries().size());
    CHECK(c.first_entry + c.entries.size() == after->entries().size());
    for (std::size_t k = 0; k < c.entries.size() && c.first_entry + k < after->entries().size(); ++k) {
        CHECK(c.entries[k] == after->entries()[c.first_entry + k]);
    }
    // Entries before first_entry are the committed ones, untouched.
    for (std::size_t k = 0; k < c.first_entry && k < before->entries().size(); ++k) {
        CHECK(before->entries()[k] == after->entries()[k]);
    }
    // The changed part starts at the first entry holding a new token (or the
    // partial tail the new tokens continue).
    CHECK(!c.entries.empty() && c.entries.front().logical_token_begin <= c.logical_token_begin);
    // The lease pins every changed page and the copy-on-write source.
    for (MappingEntry const& e : c.entries) {
        std::optional<PageMetadataSnapshot> const m = b.pageMetadata(e.handle);
        CHECK(m.has_value() && m->inflight_readers >= 1);
    }
    if (c.replaced_tail.isStructurallyValid()) {
        CHECK(c.first_entry + 1 == before->entries().size());
        CHECK(before->entries().back().handle == c.replaced_tail);
        CHECK(before->entries().back().valid_tokens == c.replaced_tokens);
        CHECK(c.entries.front().handle != c.replaced_tail);
        std::optional<PageMetadataSnapshot> const m = b.pageMetadata(c.replaced_tail);
        CHECK(m.has_value() && m->inflight_readers >= 1
              && (m->state == PageState::Sealed || m->state == PageState::Retiring));
    }
    CHECK(b.releasePageLease(c.lease_id) == KvCacheError::None);
}

void reserveStep(KvCacheManager& a, KvCacheManager& b, RequestId id, std::uint32_t expected, int finish,
                 bool lease)
{
    TokenReservationResult const r = a.reserveToken(id, expected);
    TokenReservationDelta const d = b.reserveTokenDelta(id, expected);
    CHECK(r.error == d.error);
    CHECK(r.reservation_id == d.reservation_id);
    CHECK(d.request_id == id && d.logical_token_position == expected);
    if (!r.ok() || !d.ok()) return;
    std::vector<MappingEntry> const& be = r.before.entries();
    std::vector<MappingEntry> const& re = r.reserved.entries();
    CHECK(d.committed_version == r.before.version());
    CHECK(d.entry_count == re.size());
    CHECK(d.appended == (re.size() == be.size() + 1));
    CHECK(!re.empty() && d.tail == re.back());
    CHECK(d.has_previous_tail == !be.empty());
    if (!be.empty()) CHECK(d.previous_tail == be.back());
    if (lease) {
        // The reservation lease of both managers: the candidate table and
        // the same pinned pages.
        PageLeaseAcquireResult const la = a.acquireTokenReservationLease(r.reservation_id);
        PageLeaseAcquireResult const lb = b.acquireTokenReservationLease(d.reservation_id);
        CHECK(la.error == lb.error);   // ids differ: only the delta manager leases on append
        CHECK(la.table.entries() == re && lb.table.entries() == re);
        CHECK(la.table.version() == lb.table.version() && lb.table.version() == r.reserved.version());
        CHECK(la.handles == lb.handles);
        compareRequest(a, b, id);
        if (la.ok()) CHECK(a.releasePageLease(la.lease_id) == KvCacheError::None);
        if (lb.ok()) CHECK(b.releasePageLease(lb.lease_id) == KvCacheError::None);
    }
    if (finish == 0) {
        CHECK(a.commitTokenReservation(r.reservation_id) == b.commitTokenReservation(d.reservation_id));
        std::optional<BlockTable> const t = b.blockTable(id);
        CHECK(t.has_value() && t->entries() == re && t->version() == r.reserved.version());
    } else {
        CHECK(a.rollbackTokenReservation(r.reservation_id) == b.rollbackTokenReservation(d.reservation_id));
    }
}

void run(unsigned seed)
{
    g_seed = seed;
    std::mt19937 rng(seed);
    auto pick = [&](std::uint32_t n) { return static_cast<std::uint32_t>(rng() % n); };
    std::uint32_t const micro = 24 + pick(64);
    std::uint32_t const extent = 2 + pick(6);
    KvCacheManager a(micro, extent);
    KvCacheManager b(micro, extent);
    std::uint32_t const appends[] = {1, 1, 2, 3, 5, 7, 8, 9, 15, 16, 17, 40, 64, 70};
    for (g_step = 0; g_step < 600; ++g_step) {
        RequestId const id = 1 + pick(6);
        std::optional<BlockTable> const t = a.blockTable(id);
        std::uint32_t const tokens = t ? t->tokenCount() : 0;
        switch (pick(10)) {
        case 0:
            CHECK(a.createRequest(id) == b.createRequest(id));
            break;
        case 1:
        case 2:
            appendStep(a, b, id, appends[pick(sizeof(appends) / sizeof(appends[0]))]);
            break;
        case 3:
        case 4:
        case 5:
            // Mostly the committed length; sometimes a stale one.
            reserveStep(a, b, id, pick(8) == 0 ? tokens + 1 : tokens, pick(4) == 0 ? 1 : 0, pick(3) == 0);
            break;
        case 6: {
            RequestId const child = 1 + pick(6);
            CHECK(a.forkRequest(id, child) == b.forkRequest(id, child));
            compareRequest(a, b, child);
            break;
        }
        case 7:
            CHECK(a.sealTail(id) == b.sealTail(id));
            break;
        case 8: {
            std::uint32_t const begin = 64 * pick(tokens / 64 + 1);
            PromotionPrepareResult const pa = a.preparePromotion(id, begin);
            PromotionPrepareResult const pb = b.preparePromotion(id, begin);
            CHECK(pa.error == pb.error && pa.promotion_id == pb.promotion_id);
            if (pa.ok() && pb.ok()) {
                if (pick(4) == 0) {
                    CHECK(a.rollbackPromotion(pa.promotion_id) == b.rollbackPromotion(pb.promotion_id));
                } else {
                    CHECK(a.commitPromotion(pa.promotion_id) == b.commitPromotion(pb.promotion_id));
                }
            }
            break;
        }
        default:
            if (pick(3) == 0) CHECK(a.releaseRequest(id) == b.releaseRequest(id));
            break;
        }
        compareRequest(a, b, id);
        comparePools(a, b);
    }
    for (RequestId id = 1; id <= 6; ++id) compareRequest(a, b, id);
}

}  // namespace

int main()
{
    for (unsigned seed = 1; seed <= 40; ++seed) run(seed);
    if (failures != 0) {
        std::printf("%d failures\n", failures);
        return 1;
    }
    std::printf("manager delta paths: 40 seeds x 600 steps agree\n");
    return 0;
}
