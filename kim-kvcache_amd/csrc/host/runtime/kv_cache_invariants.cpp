// KvCacheManager::checkInvariants: recount every reference, pin, reader and
// staged target from the tables, promotions, reservations and leases and
// compare with the per-page records and the pools (same predicates as
// src/runtime/kv_cache_invariants.cpp:82-497 in the reference).
#include "kim-kv/runtime/kv_cache_manager.h"

#include <algorithm>
#include <limits>

namespace kimkvcache {

struct KvCacheManager::Expected final {
    std::vector<std::uint32_t> refs[2];
    std::vector<std::uint32_t> pins[2];
    std::vector<std::uint32_t> readers[2];
    std::vector<std::uint8_t> targets[2];

    Expected(std::size_t micro, std::size_t extent)
    {
        std::size_t const n[2] = {micro, extent};
        for (int k = 0; k < 2; ++k) {
            refs[k].assign(n[k], 0);
            pins[k].assign(n[k], 0);
            readers[k].assign(n[k], 0);
            targets[k].assign(n[k], 0);
        }
    }
    static int idx(PageKind kind) { return kind == PageKind::Micro ? 0 : 1; }
};

namespace {
constexpr std::uint32_t kU32Max = std::numeric_limits<std::uint32_t>::max();
}

bool KvCacheManager::invariantsLocked() const
{
    if (!micro_pool_.checkInvariants() || !extent_pool_.checkInvariants()) return false;
    Expected expected(micro_pages_.size(), extent_pages_.size());
    return requestInvariantsLocked(expected) && promotionInvariantsLocked(expected)
        && reservationInvariantsLocked(expected) && leaseInvariantsLocked(expected)
        && poolInvariantsLocked(PageKind::Micro, expected) && poolInvariantsLocked(PageKind::Extent, expected);
}

bool KvCacheManager::reservationInvariantsLocked(Expected& expected) const
{
    if (reservation_of_.size() != reservations_.size()) return false;
    for (auto const& [id, r] : reservations_) {
        if (id == kInvalidKvTokenReservationId || r.id != id || r.request_id == kInvalidRequestId) return false;
        auto const table = tables_.find(r.request_id);
        auto const owner = reservation_of_.find(r.request_id);
        if (table == tables_.end() || owner == reservation_of_.end() || owner->second != id) return false;
        BlockTable const& before = table->second;
        if (!r.appended && before.entries().empty()) return false;
        BlockTable const candidate = candidateOf(r, before);
        if (!candidate.checkInvariants() || before.version() != r.prepared_version
            || candidate.version() != before.version() + 1 || candidate.tokenCount() != before.tokenCount() + 1) {
            return false;
        }
        if (static_cast<int>(r.staged.isStructurallyValid()) + static_cast<int>(r.existing_mutable.isStructurallyValid())
            != 1) {
            return false;
        }
        if (r.staged.isStructurallyValid()) {
            Page const* t = page(r.staged);
            auto& targets = expected.targets[0];
            if (t == nullptr || t->state != PageState::CopyTarget || t->ref_count != 0 || t->promotion_pins != 0
                || t->mutable_owner != kInvalidRequestId || r.staged.slot >= targets.size()
                || targets[r.staged.slot] != 0) {
                return false;
            }
            std::uint16_t const want = r.replaced_tail.isStructurallyValid()
                ? static_cast<std::uint16_t>(r.tail.valid_tokens - 1)
                : 0;
            if (t->valid_tokens != want) return false;
            targets[r.staged.slot] = 1;
        }
        if (r.existing_mutable.isStructurallyValid()) {
            Page const* p = page(r.existing_mutable);
            if (p == nullptr || p->state != PageState::Mutable || p->ref_count != 1
                || p->mutable_owner != r.request_id || before.entries().empty()
                || before.entries().back().handle != r.existing_mutable) {
                return false;
            }
        }
        if (r.replaced_tail.isStructurallyValid()) {
            Page const* p = page(r.replaced_tail);
            if (p == nullptr || p->state != PageState::Sealed || p->ref_count == 0 || before.entries().empty()
                || before.entries().back().handle != r.replaced_tail) {
                return false;
            }
        }
    }
    return true;
}

bool KvCacheManager::requestInvariantsLocked(Expected& expected) const
{
    for (auto const& [id, table] : tables_) {
        if (id == kInvalidRequestId || !table.checkInvariants()) return false;
        std::size_t const n = table.entries_.size();
        for (std::size_t i = 0; i < n; ++i) {
            MappingEntry const& e = table.entries_[i];
            Page const* p = page(e.handle);
            if (p == nullptr || p->state == PageState::Free || p->state == PageState::CopyTarget
                || p->state == PageState::Retiring || p->valid_tokens != e.valid_tokens || p->ref_count == 0) {
                return false;
            }
            if (p->state == PageState::Mutable) {
                if (i + 1 != n || e.kind != PageKind::Micro || p->ref_count != 1 || p->mutable_owner != id
                    || p->valid_tokens == 0 || p->valid_tokens >= kMicroPageTokenCapacity) {
                    return false;
                }
            } else if (p->state == PageState::Sealed) {
                if (p->mutable_owner != kInvalidRequestId) return false;
            } else {
                return false;
            }
            auto& refs = expected.refs[Expected::idx(e.kind)];
            if (e.handle.slot >= refs.size() || refs[e.handle.slot] == kU32Max) return false;
            ++refs[e.handle.slot];
        }
    }
    return true;
}

bool KvCacheManager::promotionInvariantsLocked(Expected& expected) const
{
    for (auto const& [id, pr] : promotions_) {
        if (id == kInvalidPromotionId || pr.id != id || pr.request_id == kInvalidRequestId
            || pr.target.kind != PageKind::Extent) {
            return false;
        }
        auto const tit = tables_.find(pr.request_id);
        if (tit == tables_.end()) return false;
        BlockTable const& table = tit->second;
        if (pr.prepared_version > table.version_) return false;
        Page const* t = page(pr.target);
        auto& ext_targets = expected.targets[1];
        if (t == nullptr || t->state != PageState::CopyTarget || t->valid_tokens != kExtentPageTokenCapacity
            || t->ref_count != 0 || t->promotion_pins != 0 || t->mutable_owner != kInvalidRequestId
            || pr.target.slot >= ext_targets.size() || ext_targets[pr.target.slot] != 0) {
            return false;
        }
        ext_targets[pr.target.slot] = 1;
        auto const first = std::find_if(table.entries_.begin(), table.entries_.end(),
                                        [&pr](MappingEntry const& e) { return e.handle == pr.sources[0]; });
        if (first == table.entries_.end()) return false;
        std::size_t const at = static_cast<std::size_t>(first - table.entries_.begin());
        if (table.entries_.size() - at < kPromotionSourcePageCount) return false;
        auto& micro_pins = expected.pins[0];
        for (std::size_t k = 0; k < kPromotionSourcePageCount; ++k) {
            PageHandle const s = pr.sources[k];
            MappingEntry const& e = table.entries_[at + k];
            Page const* p = page(s);
            std::uint64_t const expect = static_cast<std::uint64_t>(pr.logical_token_begin) + k * kMicroPageTokenCapacity;
            if (expect > kU32Max || s.kind != PageKind::Micro || e.handle != s || e.kind != PageKind::Micro
                || e.logical_token_begin != expect || e.valid_tokens != kMicroPageTokenCapacity || p == nullptr
                || p->state != PageState::Sealed || p->valid_tokens != kMicroPageTokenCapacity || p->ref_count == 0
                || p->promotion_pins == 0 || p->mutable_owner != kInvalidRequestId || s.slot >= micro_pins.size()
                || micro_pins[s.slot] != 0) {
                return false;
            }
            micro_pins[s.slot] = 1;
        }
    }
    return true;
}

bool KvCacheManager::leaseInvariantsLocked(Expected& expected) const
{
    for (auto const& [id, handles] : leases_) {
        if (id == kInvalidPageLeaseId) return false;
        for (PageHandle const h : handles) {
            Page const* p = page(h);
            auto& readers = expected.readers[Expected::idx(h.kind)];
            if (p == nullptr || p->state == PageState::Free || p->inflight_readers == 0 || h.slot >= readers.size()
                || readers[h.slot] == kU32Max) {
                return false;
            }
            ++readers[h.slot];
        }
    }
    return true;
}

bool KvCacheManager::poolInvariantsLocked(PageKind kind, Expected const& expected) const
{
    int const k = Expected::idx(kind);
    std::vector<Page> const& pages = kind == PageKind::Micro ? micro_pages_ : extent_pages_;
    PagePool const& p = kind == PageKind::Micro ? micro_pool_ : extent_pool_;
    auto const& refs = expected.refs[k];
    auto const& pins = expected.pins[k];
    auto const& readers = expected.readers[k];
    auto const& targets = expected.targets[k];
    if (pages.size() != refs.size() || pages.size() != pins.size() || pages.size() != readers.size()
        || pages.size() != targets.size()) {
        return false;
    }
    std::uint16_t const cap = pageTokenCapacity(kind);
    std::uint32_t live = 0;
    for (std::size_t i = 0; i < pages.size(); ++i) {
        Page const& pg = pages[i];
        if (pg.state == PageState::Free) {
            if (pg.valid_tokens != 0 || pg.ref_count != 0 || pg.promotion_pins != 0 || pg.inflight_readers != 0
                || pg.mutable_owner != kInvalidRequestId || refs[i] != 0 || pins[i] != 0 || readers[i] != 0
                || targets[i] != 0) {
                return false;
            }
            continue;
        }
        ++live;
        if (pg.generation == PageHandle::kInvalidGeneration) return false;
        PageHandle const h{kind, static_cast<std::uint32_t>(i), pg.generation};
        if (p.validate(h) != PagePoolError::None || pg.ref_count != refs[i] || pg.promotion_pins != pins[i]
            || pg.inflight_readers != readers[i]) {
            return false;
        }
        bool const is_target = targets[i] != 0;
        switch (pg.state) {
        case PageState::Free:
            return false;
        case PageState::Mutable:
            if (kind != PageKind::Micro || pg.ref_count != 1 || pg.valid_tokens == 0 || pg.valid_tokens >= cap
                || pg.mutable_owner == kInvalidRequestId || pg.promotion_pins != 0 || is_target) {
                return false;
            }
            break;
        case PageState::Sealed:
            if (pg.ref_count == 0 || pg.valid_tokens == 0 || pg.valid_tokens > cap
                || pg.mutable_owner != kInvalidRequestId || is_target) {
                return false;
            }
            break;
        case PageState::CopyTarget:
            if (!is_target || pg.ref_count != 0 || pg.promotion_pins != 0 || pg.mutable_owner != kInvalidRequestId) {
                return false;
            }
            if ((kind == PageKind::Extent && pg.valid_tokens != cap)
                || (kind == PageKind::Micro && pg.valid_tokens >= cap)) {
                return false;
            }
            break;
        case PageState::Retiring:
            if (pg.ref_count != 0 || pg.mutable_owner != kInvalidRequestId || is_target
                || (pg.promotion_pins == 0 && pg.inflight_readers == 0)) {
                return false;
            }
            break;
        }
    }
    PagePoolSnapshot const s = p.snapshot();
    return s.allocated_slots == live && s.capacityBalanced();
}

}  // namespace kimkvcache
