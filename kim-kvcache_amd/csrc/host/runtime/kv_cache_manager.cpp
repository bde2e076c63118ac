// KvCacheManager: page metadata for the heterogeneous KV cache.
//
// Observable behaviour (error codes and their precedence, slot and generation
// sequences, table versions, page states) follows the reference:
//   append                      src/runtime/kv_cache_append.cpp:12-258
//   reserve / commit / rollback src/runtime/token_reservation.cpp:34-330
//   seal / fork / release       src/runtime/kv_cache_lifecycle.cpp:12-195
//   promotion                   src/runtime/promotion.cpp:14-457
//   leases                      src/runtime/page_lease.cpp:9-189
//   page bookkeeping            src/runtime/kv_cache_manager.cpp:12-269
//   inspection                  src/runtime/kv_cache_inspection.cpp:12-77
// The implementation is organised around one Page record per physical slot
// and "staged" pages (CopyTarget) that only become visible at commit.
#include "kim-kv/runtime/kv_cache_manager.h"

#include <algorithm>
#include <limits>
#include <utility>

namespace kimkvcache {
namespace {

constexpr std::size_t kNoEntry = std::numeric_limits<std::size_t>::max();
constexpr std::uint32_t kU32Max = std::numeric_limits<std::uint32_t>::max();
constexpr std::uint64_t kU64Max = std::numeric_limits<std::uint64_t>::max();

}  // namespace

KvCacheManager::KvCacheManager(std::uint32_t micro_capacity, std::uint32_t extent_capacity)
    : micro_pool_(PageKind::Micro, micro_capacity),
      extent_pool_(PageKind::Extent, extent_capacity),
      micro_pages_(micro_capacity),
      extent_pages_(extent_capacity)
{
}

// ---- page bookkeeping ---------------------------------------------------------

KvCacheManager::Page* KvCacheManager::page(PageHandle h) noexcept
{
    return const_cast<Page*>(static_cast<KvCacheManager const*>(this)->page(h));
}

KvCacheManager::Page const* KvCacheManager::page(PageHandle h) const noexcept
{
    if (!h.isStructurallyValid()) return nullptr;
    std::vector<Page> const& pages = h.kind == PageKind::Micro ? micro_pages_ : extent_pages_;
    if (h.slot >= pages.size()) return nullptr;
    Page const& p = pages[h.slot];
    return p.generation == h.generation ? &p : nullptr;
}

void KvCacheManager::clearFreed(Page& p) noexcept
{
    // The generation stays: it identifies the slot's last handle.
    p.state = PageState::Free;
    p.valid_tokens = 0;
    p.ref_count = 0;
    p.promotion_pins = 0;
    p.inflight_readers = 0;
    p.mutable_owner = kInvalidRequestId;
}

KvCacheError KvCacheManager::stageMicroLocked(std::uint16_t initial_valid_tokens, PageHandle& out)
{
    if (initial_valid_tokens >= kMicroPageTokenCapacity) return KvCacheError::InvalidArgument;
    PageAllocationResult const a = micro_pool_.allocate();
    if (!a.ok()) {
        return a.error == PagePoolError::Exhausted ? KvCacheError::ResourceExhausted
                                                   : KvCacheError::InternalInvariantViolation;
    }
    out = a.handle;
    if (out.slot >= micro_pages_.size()) {
        static_cast<void>(micro_pool_.release(out));
        out = PageHandle::invalid();
        return KvCacheError::InternalInvariantViolation;
    }
    Page& p = micro_pages_[out.slot];
    if (p.state != PageState::Free || p.ref_count != 0 || p.promotion_pins != 0 || p.inflight_readers != 0) {
        static_cast<void>(micro_pool_.release(out));
        out = PageHandle::invalid();
        return KvCacheError::InternalInvariantViolation;
    }
    p = Page{PageState::CopyTarget, out.generation, initial_valid_tokens, 0, 0, 0, kInvalidRequestId};
    return KvCacheError::None;
}

KvCacheError KvCacheManager::stageExtentLocked(PageHandle& out)
{
    PageAllocationResult const a = extent_pool_.allocate();
    if (!a.ok()) {
        return a.error == PagePoolError::Exhausted ? KvCacheError::ResourceExhausted
                                                   : KvCacheError::InternalInvariantViolation;
    }
    out = a.handle;
    if (out.slot >= extent_pages_.size()) {
        static_cast<void>(extent_pool_.release(out));
        out = PageHandle::invalid();
        return KvCacheError::InternalInvariantViolation;
    }
    Page& p = extent_pages_[out.slot];
    if (p.state != PageState::Free || p.ref_count != 0 || p.promotion_pins != 0 || p.inflight_readers != 0) {
        static_cast<void>(extent_pool_.release(out));
        out = PageHandle::invalid();
        return KvCacheError::InternalInvariantViolation;
    }
    p = Page{PageState::CopyTarget, out.generation, kExtentPageTokenCapacity, 0, 0, 0, kInvalidRequestId};
    return KvCacheError::None;
}

void KvCacheManager::unstageLocked(std::vector<Staged> const& staged) noexcept
{
    for (auto it = staged.rbegin(); it != staged.rend(); ++it) {
        Page* p = page(it->handle);
        if (p == nullptr || p->state != PageState::CopyTarget || p->ref_count != 0) continue;
        if (micro_pool_.release(it->handle) == PagePoolError::None) clearFreed(*p);
    }
}

KvCacheError KvCacheManager::freeLocked(PageHandle h)
{
    Page* p = page(h);
    if (p == nullptr || p->state == PageState::Free) return KvCacheError::InternalInvariantViolation;
    if (p->ref_count != 0) return KvCacheError::InvalidState;
    p->mutable_owner = kInvalidRequestId;
    if (p->promotion_pins != 0 || p->inflight_readers != 0) {
        p->state = PageState::Retiring;     // returns to the pool when unpinned
        return KvCacheError::None;
    }
    PagePool& owner = pool(h.kind);
    if (owner.validate(h) != PagePoolError::None || owner.release(h) != PagePoolError::None) {
        return KvCacheError::InternalInvariantViolation;
    }
    clearFreed(*p);
    return KvCacheError::None;
}

KvCacheError KvCacheManager::dropReferenceLocked(PageHandle h)
{
    Page* p = page(h);
    if (p == nullptr || p->state == PageState::Free || p->state == PageState::CopyTarget || p->ref_count == 0) {
        return KvCacheError::InternalInvariantViolation;
    }
    if (--p->ref_count != 0) return KvCacheError::None;
    return freeLocked(h);
}

template <typename Map>
std::uint64_t KvCacheManager::nextId(std::uint64_t& counter, Map const& live)
{
    // Among N live ids, N+1 consecutive candidates always contain a free one.
    for (std::size_t attempt = 0; attempt < live.size() + 1; ++attempt) {
        std::uint64_t const candidate = counter++;
        if (counter == 0) counter = 1;
        if (candidate != 0 && live.find(candidate) == live.end()) return candidate;
    }
    return 0;
}

bool KvCacheManager::hasReservationLocked(RequestId request_id) const noexcept
{
    return reservation_of_.find(request_id) != reservation_of_.end();
}

// ---- requests -------------------------------------------------------------------

KvCacheError KvCacheManager::createRequest(RequestId request_id)
{
    if (request_id == kInvalidRequestId) return KvCacheError::InvalidArgument;
    std::lock_guard<std::mutex> lock(mutex_);
    return tables_.emplace(request_id, BlockTable{}).second ? KvCacheError::None
                                                            : KvCacheError::RequestAlreadyExists;
}

KvCacheError KvCacheManager::append(RequestId request_id, std::uint32_t token_count)
{
    if (request_id == kInvalidRequestId || token_count == 0) return KvCacheError::InvalidArgument;
    std::lock_guard<std::mutex> lock(mutex_);
    return appendLocked(request_id, token_count, nullptr);
}

AppendChange KvCacheManager::appendWithLease(RequestId request_id, std::uint32_t token_count)
{
    AppendChange change;
    if (request_id == kInvalidRequestId || token_count == 0) {
        change.error = KvCacheError::InvalidArgument;
        return change;
    }
    std::lock_guard<std::mutex> lock(mutex_);
    change.error = appendLocked(request_id, token_count, &change);
    return change;
}

KvCacheError KvCacheManager::appendLocked(RequestId request_id, std::uint32_t token_count, AppendChange* change)
{
    auto it = tables_.find(request_id);
    if (it == tables_.end()) return KvCacheError::RequestNotFound;
    if (hasReservationLocked(request_id)) return KvCacheError::RequestConflict;
    BlockTable& table = it->second;
    std::uint32_t const old_tokens = table.tokenCount();
    if (token_count > kU32Max - old_tokens) return KvCacheError::InvalidArgument;

    // Only the table's end changes: `part` replaces its entries from `first`
    // on -- the partial micro tail, when there is one (extended in place, or
    // continued in a private copy when it is sealed), then fresh pages.
    std::size_t const max_new = (static_cast<std::size_t>(token_count) + kMicroPageTokenCapacity - 1)
            / kMicroPageTokenCapacity + 1;
    table.entries_.reserve(table.entries_.size() + max_new);   // so that the commit cannot fail on memory
    std::size_t first = table.entries_.size();
    std::vector<MappingEntry> part;
    part.reserve(max_new);
    std::vector<Staged> staged;   // entry: index in the new table
    staged.reserve(max_new);

    std::size_t active = kNoEntry;   // index in `part` of the page taking tokens
    PageHandle existing_mutable = PageHandle::invalid();
    PageHandle replaced_tail = PageHandle::invalid();
    std::uint16_t replaced_tokens = 0;

    if (!table.entries_.empty()) {
        MappingEntry tail = table.entries_.back();
        Page* tp = page(tail.handle);
        if (tp == nullptr || tp->valid_tokens != tail.valid_tokens) return KvCacheError::InternalInvariantViolation;
        if (tail.kind == PageKind::Micro && tail.valid_tokens < kMicroPageTokenCapacity) {
            first = table.entries_.size() - 1;
            if (tp->state == PageState::Mutable) {
                if (tp->ref_count != 1 || tp->mutable_owner != request_id) {
                    return KvCacheError::InternalInvariantViolation;
                }
                existing_mutable = tail.handle;
            } else if (tp->state == PageState::Sealed) {
                // Shared or sealed partial tail: continue in a private copy.
                PageHandle copy = PageHandle::invalid();
                KvCacheError const e = stageMicroLocked(tail.valid_tokens, copy);
                if (e != KvCacheError::None) return e;
                staged.push_back(Staged{copy, first});
                replaced_tail = tail.handle;
                replaced_tokens = tail.valid_tokens;
                tail.handle = copy;
            } else {
                return KvCacheError::InvalidState;
            }
            part.push_back(tail);
            active = 0;
        } else if (tp->state != PageState::Sealed) {
            return KvCacheError::InternalInvariantViolation;
        }
    }

    std::uint32_t remaining = token_count;
    std::uint32_t logical_end = old_tokens;
    while (remaining != 0) {
        if (active == kNoEntry) {
            PageHandle fresh = PageHandle::invalid();
            KvCacheError const e = stageMicroLocked(0, fresh);
            if (e != KvCacheError::None) {
                unstageLocked(staged);
                return e;
            }
            part.push_back(MappingEntry{logical_end, 0, PageKind::Micro, fresh});
            active = part.size() - 1;
            staged.push_back(Staged{fresh, first + active});
        }
        MappingEntry& a = part[active];
        std::uint32_t const take = std::min<std::uint32_t>(remaining, kMicroPageTokenCapacity - a.valid_tokens);
        a.valid_tokens = static_cast<std::uint16_t>(a.valid_tokens + take);
        logical_end += take;
        remaining -= take;
        if (a.valid_tokens == kMicroPageTokenCapacity) active = kNoEntry;
    }

    auto fail = [&](KvCacheError e) {
        unstageLocked(staged);
        return e;
    };
    if (change == nullptr) {
        BlockTable cand = table;
        cand.entries_.resize(first);
        cand.entries_.insert(cand.entries_.end(), part.begin(), part.end());
        cand.version_ = table.version_ + 1;
        if (!cand.checkInvariants()) return fail(KvCacheError::InternalInvariantViolation);
    } else {
        // The committed table satisfies the table invariants and a staged
        // page is in no table, so checking the replaced end (contiguous with
        // the kept entries, micro pages of 1..8 tokens) checks the candidate.
        std::uint32_t next = first < table.entries_.size() ? table.entries_[first].logical_token_begin : old_tokens;
        for (MappingEntry const& e : part) {
            if (!e.handle.isStructurallyValid() || e.handle.kind != PageKind::Micro || e.kind != PageKind::Micro
                || e.logical_token_begin != next || e.valid_tokens == 0 || e.valid_tokens > kMicroPageTokenCapacity) {
                return fail(KvCacheError::InternalInvariantViolation);
            }
            next += e.valid_tokens;
        }
        if (next != logical_end) return fail(KvCacheError::InternalInvariantViolation);
    }
    if (existing_mutable.isStructurallyValid()) {
        Page* p = page(existing_mutable);
        if (p == nullptr || p->state != PageState::Mutable || p->ref_count != 1 || p->mutable_owner != request_id) {
            return fail(KvCacheError::InternalInvariantViolation);
        }
    }
    if (replaced_tail.isStructurallyValid()) {
        Page* p = page(replaced_tail);
        if (p == nullptr || p->state != PageState::Sealed || p->ref_count == 0) {
            return fail(KvCacheError::InternalInvariantViolation);
        }
    }
    for (Staged const& s : staged) {
        Page* p = page(s.handle);
        if (p == nullptr || p->state != PageState::CopyTarget || p->ref_count != 0 || s.entry < first
            || s.entry - first >= part.size() || part[s.entry - first].handle != s.handle) {
            return fail(KvCacheError::InternalInvariantViolation);
        }
    }

    // The device copy's lease, taken before the replaced tail loses this
    // table's reference so that a copy-on-write source outlives the copy.
    PageLeaseId lease = kInvalidPageLeaseId;
    std::vector<PageHandle> const* leased = nullptr;
    if (change != nullptr) {
        std::vector<PageHandle> handles;
        handles.reserve(part.size() + 1);
        for (MappingEntry const& e : part) handles.push_back(e.handle);
        if (replaced_tail.isStructurallyValid()) handles.push_back(replaced_tail);
        for (PageHandle const h : handles) {
            if (page(h)->inflight_readers == kU32Max) return fail(KvCacheError::InvalidState);
        }
        lease = nextId(next_lease_id_, leases_);
        if (lease == kInvalidPageLeaseId) return fail(KvCacheError::InternalInvariantViolation);
        auto inserted = leases_.emplace(lease, std::move(handles));
        if (!inserted.second) return fail(KvCacheError::InternalInvariantViolation);
        leased = &inserted.first->second;
        for (PageHandle const h : *leased) ++page(h)->inflight_readers;
    }

    // Commit: nothing below can fail except an inconsistent replaced tail.
    if (replaced_tail.isStructurallyValid()) {
        KvCacheError const e = dropReferenceLocked(replaced_tail);
        if (e != KvCacheError::None) {
            if (leased != nullptr) {
                for (PageHandle const h : *leased) --page(h)->inflight_readers;
                leases_.erase(lease);
            }
            return fail(e);
        }
    }
    if (existing_mutable.isStructurallyValid()) {
        Page* p = page(existing_mutable);
        MappingEntry const& e = part.front();   // the extended tail
        p->valid_tokens = e.valid_tokens;
        if (e.valid_tokens == kMicroPageTokenCapacity) {
            p->state = PageState::Sealed;
            p->mutable_owner = kInvalidRequestId;
        }
    }
    for (Staged const& s : staged) {
        Page* p = page(s.handle);
        MappingEntry const& e = part[s.entry - first];
        p->valid_tokens = e.valid_tokens;
        p->ref_count = 1;
        bool const full = e.valid_tokens == kMicroPageTokenCapacity;
        p->state = full ? PageState::Sealed : PageState::Mutable;
        p->mutable_owner = full ? kInvalidRequestId : request_id;
    }
    table.entries_.resize(first);
    table.entries_.insert(table.entries_.end(), part.begin(), part.end());
    ++table.version_;
    if (change != nullptr) {
        change->logical_token_begin = old_tokens;
        change->version = table.version_;
        change->first_entry = first;
        change->entries = std::move(part);
        change->replaced_tail = replaced_tail;
        change->replaced_tokens = replaced_tokens;
        change->lease_id = lease;
    }
    return KvCacheError::None;
}

// ---- single-token reservations --------------------------------------------------

TokenReservationDelta KvCacheManager::reserveLocked(RequestId request_id, std::uint32_t expected_committed_tokens,
                                                    BlockTable* candidate)
{
    TokenReservationDelta out;
    out.request_id = request_id;
    out.logical_token_position = expected_committed_tokens;
    auto it = tables_.find(request_id);
    if (it == tables_.end()) {
        out.error = KvCacheError::RequestNotFound;
        return out;
    }
    bool const promoting = std::any_of(promotions_.begin(), promotions_.end(),
                                       [request_id](auto const& p) { return p.second.request_id == request_id; });
    if (hasReservationLocked(request_id) || promoting) {
        out.error = KvCacheError::RequestConflict;
        return out;
    }
    BlockTable& before = it->second;
    if (before.tokenCount() != expected_committed_tokens || before.version_ == kU64Max
        || expected_committed_tokens == kU32Max) {
        out.error = KvCacheError::InvalidState;
        return out;
    }
    // A new entry is appended when there is no partial micro tail; the
    // committed table gets the room now so that commit cannot fail on memory.
    bool const appended = before.entries_.empty() || before.entries_.back().kind == PageKind::Extent
        || before.entries_.back().valid_tokens == kMicroPageTokenCapacity;
    if (appended) before.entries_.reserve(before.entries_.size() + 1);

    PageHandle staged = PageHandle::invalid();
    PageHandle existing_mutable = PageHandle::invalid();
    PageHandle replaced_tail = PageHandle::invalid();
    MappingEntry tail{};
    if (appended) {
        KvCacheError const e = stageMicroLocked(0, staged);
        if (e != KvCacheError::None) {
            out.error = e;
            return out;
        }
        tail = MappingEntry{expected_committed_tokens, 1, PageKind::Micro, staged};
    } else {
        tail = before.entries_.back();
        Page* p = page(tail.handle);
        if (p == nullptr || tail.kind != PageKind::Micro || p->valid_tokens != tail.valid_tokens) {
            out.error = KvCacheError::InternalInvariantViolation;
            return out;
        }
        if (p->state == PageState::Mutable) {
            if (p->ref_count != 1 || p->mutable_owner != request_id) {
                out.error = KvCacheError::InternalInvariantViolation;
                return out;
            }
            existing_mutable = tail.handle;
        } else if (p->state == PageState::Sealed) {
            // Copy-on-write: the shared partial tail is replaced by a fresh page.
            KvCacheError const e = stageMicroLocked(tail.valid_tokens, staged);
            if (e != KvCacheError::None) {
                out.error = e;
                return out;
            }
            replaced_tail = tail.handle;
            tail.handle = staged;
        } else {
            out.error = KvCacheError::InvalidState;
            return out;
        }
        ++tail.valid_tokens;
    }

    auto abandon = [&](KvCacheError e) {
        if (staged.isStructurallyValid()) static_cast<void>(freeLocked(staged));
        out.error = e;
        return out;
    };
    bool sound = false;
    if (candidate != nullptr) {
        Reservation const probe{0, request_id, before.version_, tail, appended, staged, existing_mutable,
                                replaced_tail};
        *candidate = candidateOf(probe, before);
        sound = candidate->checkInvariants();
    } else {
        // The committed table satisfies the table invariants; only its tail
        // changed, and a staged page is in no table, so checking the tail
        // entry checks the candidate.
        std::uint32_t const begin = appended ? before.tokenCount() : before.entries_.back().logical_token_begin;
        sound = tail.handle.isStructurallyValid() && tail.handle.kind == PageKind::Micro
            && tail.logical_token_begin == begin && tail.valid_tokens >= 1
            && tail.valid_tokens <= kMicroPageTokenCapacity;
    }
    if (!sound) return abandon(KvCacheError::InternalInvariantViolation);
    KvTokenReservationId const id = nextId(next_reservation_id_, reservations_);
    if (id == kInvalidKvTokenReservationId) return abandon(KvCacheError::InternalInvariantViolation);
    auto inserted = reservations_.emplace(
        id, Reservation{id, request_id, before.version_, tail, appended, staged, existing_mutable, replaced_tail});
    if (!inserted.second) return abandon(KvCacheError::InternalInvariantViolation);
    if (!reservation_of_.emplace(request_id, id).second) {
        reservations_.erase(inserted.first);
        return abandon(KvCacheError::InternalInvariantViolation);
    }
    out.error = KvCacheError::None;
    out.reservation_id = id;
    out.committed_version = before.version_;
    out.entry_count = static_cast<std::uint32_t>(before.entries_.size() + (appended ? 1 : 0));
    out.appended = appended;
    out.has_previous_tail = !before.entries_.empty();
    if (out.has_previous_tail) out.previous_tail = before.entries_.back();
    out.tail = tail;
    return out;
}

BlockTable KvCacheManager::candidateOf(Reservation const& r, BlockTable const& committed)
{
    BlockTable cand = committed;
    if (r.appended) {
        cand.entries_.push_back(r.tail);
    } else if (!cand.entries_.empty()) {
        cand.entries_.back() = r.tail;
    }
    cand.version_ = r.prepared_version + 1;
    return cand;
}

TokenReservationResult KvCacheManager::reserveToken(RequestId request_id, std::uint32_t expected_committed_tokens)
{
    TokenReservationResult result;
    result.request_id = request_id;
    result.logical_token_position = expected_committed_tokens;
    if (request_id == kInvalidRequestId) {
        result.error = KvCacheError::InvalidArgument;
        return result;
    }
    std::lock_guard<std::mutex> lock(mutex_);
    BlockTable cand;
    TokenReservationDelta const d = reserveLocked(request_id, expected_committed_tokens, &cand);
    result.error = d.error;
    if (!d.ok()) return result;
    result.reservation_id = d.reservation_id;
    result.before = tables_.find(request_id)->second;
    result.reserved = std::move(cand);
    return result;
}

TokenReservationDelta KvCacheManager::reserveTokenDelta(RequestId request_id,
                                                        std::uint32_t expected_committed_tokens)
{
    if (request_id == kInvalidRequestId) {
        TokenReservationDelta out;
        out.request_id = request_id;
        out.logical_token_position = expected_committed_tokens;
        out.error = KvCacheError::InvalidArgument;
        return out;
    }
    std::lock_guard<std::mutex> lock(mutex_);
    return reserveLocked(request_id, expected_committed_tokens, nullptr);
}

KvCacheError KvCacheManager::commitTokenReservation(KvTokenReservationId reservation_id)
{
    if (reservation_id == kInvalidKvTokenReservationId) return KvCacheError::InvalidArgument;
    std::lock_guard<std::mutex> lock(mutex_);
    auto rit = reservations_.find(reservation_id);
    if (rit == reservations_.end()) return KvCacheError::TokenReservationNotFound;
    Reservation& r = rit->second;
    auto tit = tables_.find(r.request_id);
    if (tit == tables_.end() || tit->second.version_ != r.prepared_version) return KvCacheError::RequestConflict;

    MappingEntry const& tail = r.tail;
    BlockTable& table = tit->second;
    if (!r.appended && table.entries_.empty()) return KvCacheError::InternalInvariantViolation;
    Page* staged = r.staged.isStructurallyValid() ? page(r.staged) : nullptr;
    Page* existing = r.existing_mutable.isStructurallyValid() ? page(r.existing_mutable) : nullptr;
    Page* replaced = r.replaced_tail.isStructurallyValid() ? page(r.replaced_tail) : nullptr;
    if ((staged != nullptr && (staged->state != PageState::CopyTarget || staged->ref_count != 0))
        || (existing != nullptr
            && (existing->state != PageState::Mutable || existing->ref_count != 1
                || existing->mutable_owner != r.request_id))
        || (replaced != nullptr && (replaced->state != PageState::Sealed || replaced->ref_count == 0))) {
        return KvCacheError::InternalInvariantViolation;
    }
    if (r.replaced_tail.isStructurallyValid()) {
        KvCacheError const e = dropReferenceLocked(r.replaced_tail);
        if (e != KvCacheError::None) return e;
    }
    bool const full = tail.valid_tokens == kMicroPageTokenCapacity;
    if (existing != nullptr) {
        existing->valid_tokens = tail.valid_tokens;
        if (full) {
            existing->state = PageState::Sealed;
            existing->mutable_owner = kInvalidRequestId;
        }
    }
    if (staged != nullptr) {
        staged->valid_tokens = tail.valid_tokens;
        staged->ref_count = 1;
        staged->state = full ? PageState::Sealed : PageState::Mutable;
        staged->mutable_owner = full ? kInvalidRequestId : r.request_id;
    }
    // The candidate: the committed table with the new tail (room for an
    // appended entry was reserved with the reservation).
    if (r.appended) {
        table.entries_.push_back(tail);
    } else {
        table.entries_.back() = tail;
    }
    table.version_ = r.prepared_version + 1;
    reservation_of_.erase(r.request_id);
    reservations_.erase(rit);
    return KvCacheError::None;
}

KvCacheError KvCacheManager::rollbackReservationLocked(KvTokenReservationId reservation_id)
{
    auto it = reservations_.find(reservation_id);
    if (it == reservations_.end()) return KvCacheError::TokenReservationNotFound;
    if (it->second.staged.isStructurallyValid()) {
        KvCacheError const e = freeLocked(it->second.staged);
        if (e != KvCacheError::None) return e;
    }
    reservation_of_.erase(it->second.request_id);
    reservations_.erase(it);
    return KvCacheError::None;
}

KvCacheError KvCacheManager::rollbackTokenReservation(KvTokenReservationId reservation_id)
{
    if (reservation_id == kInvalidKvTokenReservationId) return KvCacheError::InvalidArgument;
    std::lock_guard<std::mutex> lock(mutex_);
    return rollbackReservationLocked(reservation_id);
}

PageLeaseAcquireResult KvCacheManager::acquireTokenReservationLease(KvTokenReservationId reservation_id)
{
    PageLeaseAcquireResult result;
    if (reservation_id == kInvalidKvTokenReservationId) {
        result.error = KvCacheError::InvalidArgument;
        return result;
    }
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = reservations_.find(reservation_id);
    if (it == reservations_.end()) {
        result.error = KvCacheError::TokenReservationNotFound;
        return result;
    }
    Reservation const& r = it->second;
    auto const committed = tables_.find(r.request_id);
    if (committed == tables_.end()) {
        result.error = KvCacheError::InternalInvariantViolation;
        return result;
    }
    BlockTable cand = candidateOf(r, committed->second);
    std::vector<PageHandle> handles;
    handles.reserve(cand.entries_.size() + 1);
    for (MappingEntry const& e : cand.entries_) handles.push_back(e.handle);
    if (r.replaced_tail.isStructurallyValid()) handles.push_back(r.replaced_tail);
    return leaseLocked(std::move(handles), std::move(cand));
}

// ---- fork / seal / release ---------------------------------------------------------

KvCacheError KvCacheManager::sealTail(RequestId request_id)
{
    if (request_id == kInvalidRequestId) return KvCacheError::InvalidArgument;
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = tables_.find(request_id);
    if (it == tables_.end()) return KvCacheError::RequestNotFound;
    if (hasReservationLocked(request_id)) return KvCacheError::RequestConflict;
    BlockTable& table = it->second;
    if (table.entries_.empty()) return KvCacheError::InvalidState;
    MappingEntry const& tail = table.entries_.back();
    Page* p = page(tail.handle);
    if (p == nullptr || p->valid_tokens != tail.valid_tokens) return KvCacheError::InternalInvariantViolation;
    if (p->state == PageState::Sealed) return KvCacheError::None;
    if (p->state != PageState::Mutable || p->ref_count != 1 || p->mutable_owner != request_id) {
        return KvCacheError::InvalidState;
    }
    p->state = PageState::Sealed;           // mapping unchanged: no version bump
    p->mutable_owner = kInvalidRequestId;
    return KvCacheError::None;
}

KvCacheError KvCacheManager::forkRequest(RequestId source_request_id, RequestId child_request_id)
{
    if (source_request_id == kInvalidRequestId || child_request_id == kInvalidRequestId
        || source_request_id == child_request_id) {
        return KvCacheError::InvalidArgument;
    }
    std::lock_guard<std::mutex> lock(mutex_);
    auto sit = tables_.find(source_request_id);
    if (sit == tables_.end()) return KvCacheError::RequestNotFound;
    if (hasReservationLocked(source_request_id)) return KvCacheError::RequestConflict;
    if (tables_.find(child_request_id) != tables_.end()) return KvCacheError::RequestAlreadyExists;
    BlockTable const& source = sit->second;
    std::size_t const n = source.entries_.size();
    for (std::size_t i = 0; i < n; ++i) {
        MappingEntry const& e = source.entries_[i];
        Page const* p = page(e.handle);
        if (p == nullptr || p->valid_tokens != e.valid_tokens || p->ref_count == 0 || p->ref_count == kU32Max) {
            return KvCacheError::InternalInvariantViolation;
        }
        if (p->state == PageState::Mutable) {
            if (i + 1 != n || p->ref_count != 1 || p->mutable_owner != source_request_id) {
                return KvCacheError::InternalInvariantViolation;
            }
        } else if (p->state != PageState::Sealed) {
            return KvCacheError::InvalidState;
        }
    }
    BlockTable child = source;
    child.version_ = child.entries_.empty() ? 0 : 1;   // independent version history
    auto inserted = tables_.emplace(child_request_id, std::move(child));
    if (!inserted.second) return KvCacheError::RequestAlreadyExists;
    for (MappingEntry const& e : source.entries_) {
        Page* p = page(e.handle);
        if (p->state == PageState::Mutable) {
            p->state = PageState::Sealed;
            p->mutable_owner = kInvalidRequestId;
        }
        ++p->ref_count;
    }
    return KvCacheError::None;
}

KvCacheError KvCacheManager::releaseRequest(RequestId request_id)
{
    if (request_id == kInvalidRequestId) return KvCacheError::InvalidArgument;
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = tables_.find(request_id);
    if (it == tables_.end()) return KvCacheError::RequestNotFound;
    if (hasReservationLocked(request_id)) return KvCacheError::RequestConflict;
    KvCacheError const rb = rollbackRequestPromotionsLocked(request_id);
    if (rb != KvCacheError::None) return rb;
    for (MappingEntry const& e : it->second.entries_) {
        Page const* p = page(e.handle);
        if (p == nullptr || p->state == PageState::Free || p->state == PageState::CopyTarget || p->ref_count == 0) {
            return KvCacheError::InternalInvariantViolation;
        }
    }
    for (MappingEntry const& e : it->second.entries_) {
        KvCacheError const d = dropReferenceLocked(e.handle);
        if (d != KvCacheError::None) return d;
    }
    tables_.erase(it);
    return KvCacheError::None;
}

// ---- promotion --------------------------------------------------------------------

PromotionPrepareResult KvCacheManager::preparePromotion(RequestId request_id, std::uint32_t logical_token_begin)
{
    PromotionPrepareResult result;
    result.request_id = request_id;
    result.logical_token_begin = logical_token_begin;
    if (request_id == kInvalidRequestId) {
        result.error = KvCacheError::InvalidArgument;
        return result;
    }
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = tables_.find(request_id);
    if (it == tables_.end()) {
        result.error = KvCacheError::RequestNotFound;
        return result;
    }
    if (hasReservationLocked(request_id)) {
        result.error = KvCacheError::RequestConflict;
        return result;
    }
    BlockTable const& table = it->second;
    if (table.version_ == kU64Max) {
        result.error = KvCacheError::PromotionConflict;
        return result;
    }
    auto first = std::find_if(table.entries_.begin(), table.entries_.end(), [logical_token_begin](auto const& e) {
        return e.logical_token_begin == logical_token_begin;
    });
    std::size_t const idx = static_cast<std::size_t>(first - table.entries_.begin());
    if (first == table.entries_.end() || table.entries_.size() - idx < kPromotionSourcePageCount) {
        result.error = KvCacheError::PromotionNotEligible;
        return result;
    }
    std::array<PageHandle, kPromotionSourcePageCount> sources{};
    for (std::size_t k = 0; k < kPromotionSourcePageCount; ++k) {
        MappingEntry const& e = table.entries_[idx + k];
        std::uint64_t const expect = static_cast<std::uint64_t>(logical_token_begin) + k * kMicroPageTokenCapacity;
        Page const* p = page(e.handle);
        bool const eligible = expect <= kU32Max && e.logical_token_begin == expect && e.kind == PageKind::Micro
            && e.handle.kind == PageKind::Micro && e.valid_tokens == kMicroPageTokenCapacity && p != nullptr
            && p->state == PageState::Sealed && p->valid_tokens == kMicroPageTokenCapacity && p->ref_count == 1
            && p->promotion_pins == 0 && p->mutable_owner == kInvalidRequestId
            && micro_pool_.validate(e.handle) == PagePoolError::None;
        if (!eligible) {
            result.error = KvCacheError::PromotionNotEligible;
            return result;
        }
        sources[k] = e.handle;
    }
    PageHandle target = PageHandle::invalid();
    KvCacheError const e = stageExtentLocked(target);
    if (e != KvCacheError::None) {
        result.error = e;
        return result;
    }
    PromotionId const id = nextId(next_promotion_id_, promotions_);
    if (id == kInvalidPromotionId) {
        static_cast<void>(freeLocked(target));
        result.error = KvCacheError::InternalInvariantViolation;
        return result;
    }
    if (!promotions_.emplace(id, Promotion{id, request_id, table.version_, logical_token_begin, idx, sources, target})
             .second) {
        static_cast<void>(freeLocked(target));
        result.error = KvCacheError::InternalInvariantViolation;
        return result;
    }
    for (PageHandle const s : sources) ++page(s)->promotion_pins;
    result.error = KvCacheError::None;
    result.promotion_id = id;
    result.source_handles = sources;
    result.target_handle = target;
    return result;
}

KvCacheError KvCacheManager::rollbackPromotionLocked(PromotionId promotion_id)
{
    auto it = promotions_.find(promotion_id);
    if (it == promotions_.end()) return KvCacheError::PromotionNotFound;
    Promotion const& pr = it->second;
    Page const* t = page(pr.target);
    if (t == nullptr || t->state != PageState::CopyTarget || t->valid_tokens != kExtentPageTokenCapacity
        || t->ref_count != 0 || t->promotion_pins != 0 || t->mutable_owner != kInvalidRequestId
        || extent_pool_.validate(pr.target) != PagePoolError::None) {
        return KvCacheError::InternalInvariantViolation;
    }
    for (PageHandle const s : pr.sources) {
        Page const* p = page(s);
        if (p == nullptr || (p->state != PageState::Sealed && p->state != PageState::Retiring)
            || p->valid_tokens != kMicroPageTokenCapacity || p->promotion_pins != 1
            || p->mutable_owner != kInvalidRequestId || micro_pool_.validate(s) != PagePoolError::None) {
            return KvCacheError::InternalInvariantViolation;
        }
    }
    KvCacheError const e = freeLocked(pr.target);
    if (e != KvCacheError::None) return e;
    for (PageHandle const s : pr.sources) {
        Page* p = page(s);
        --p->promotion_pins;
        if (p->ref_count == 0) {
            KvCacheError const f = freeLocked(s);
            if (f != KvCacheError::None) return f;
        }
    }
    promotions_.erase(it);
    return KvCacheError::None;
}

KvCacheError KvCacheManager::rollbackPromotion(PromotionId promotion_id)
{
    if (promotion_id == kInvalidPromotionId) return KvCacheError::InvalidArgument;
    std::lock_guard<std::mutex> lock(mutex_);
    return rollbackPromotionLocked(promotion_id);
}

KvCacheError KvCacheManager::rollbackRequestPromotionsLocked(RequestId request_id)
{
    for (;;) {
        auto it = std::find_if(promotions_.begin(), promotions_.end(),
                               [request_id](auto const& p) { return p.second.request_id == request_id; });
        if (it == promotions_.end()) return KvCacheError::None;
        KvCacheError const e = rollbackPromotionLocked(it->first);
        if (e != KvCacheError::None) return e;
    }
}

KvCacheError KvCacheManager::commitPromotion(PromotionId promotion_id)
{
    if (promotion_id == kInvalidPromotionId) return KvCacheError::InvalidArgument;
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = promotions_.find(promotion_id);
    if (it == promotions_.end()) return KvCacheError::PromotionNotFound;
    Promotion const pr = it->second;
    auto abort_with = [this, promotion_id](KvCacheError e) {
        KvCacheError const r = rollbackPromotionLocked(promotion_id);
        return r == KvCacheError::None ? e : r;
    };
    auto tit = tables_.find(pr.request_id);
    if (tit == tables_.end()) return abort_with(KvCacheError::PromotionConflict);
    BlockTable& table = tit->second;
    if (table.version_ != pr.prepared_version || pr.first_entry > table.entries_.size()
        || table.entries_.size() - pr.first_entry < kPromotionSourcePageCount || table.version_ == kU64Max) {
        return abort_with(KvCacheError::PromotionConflict);
    }
    Page* t = page(pr.target);
    if (t == nullptr || t->state != PageState::CopyTarget || t->valid_tokens != kExtentPageTokenCapacity
        || t->ref_count != 0 || t->promotion_pins != 0 || t->inflight_readers != 0
        || t->mutable_owner != kInvalidRequestId || extent_pool_.validate(pr.target) != PagePoolError::None) {
        return abort_with(KvCacheError::PromotionConflict);
    }
    for (std::size_t k = 0; k < kPromotionSourcePageCount; ++k) {
        MappingEntry const& e = table.entries_[pr.first_entry + k];
        PageHandle const s = pr.sources[k];
        Page const* p = page(s);
        std::uint64_t const expect = static_cast<std::uint64_t>(pr.logical_token_begin) + k * kMicroPageTokenCapacity;
        bool const same = expect <= kU32Max && e.logical_token_begin == expect && e.kind == PageKind::Micro
            && e.valid_tokens == kMicroPageTokenCapacity && e.handle == s && p != nullptr
            && p->state == PageState::Sealed && p->valid_tokens == kMicroPageTokenCapacity && p->ref_count == 1
            && p->promotion_pins == 1 && p->mutable_owner == kInvalidRequestId
            && micro_pool_.validate(s) == PagePoolError::None;
        if (!same) return abort_with(KvCacheError::PromotionConflict);
    }
    BlockTable cand = table;
    auto const first = cand.entries_.begin() + static_cast<std::ptrdiff_t>(pr.first_entry);
    *first = MappingEntry{pr.logical_token_begin, kExtentPageTokenCapacity, PageKind::Extent, pr.target};
    cand.entries_.erase(first + 1, first + static_cast<std::ptrdiff_t>(kPromotionSourcePageCount));
    cand.version_ = table.version_ + 1;
    if (!cand.checkInvariants()) return abort_with(KvCacheError::InternalInvariantViolation);

    table = std::move(cand);
    t->state = PageState::Sealed;
    t->ref_count = 1;
    for (PageHandle const s : pr.sources) {
        Page* p = page(s);
        --p->ref_count;
        --p->promotion_pins;
        KvCacheError const e = freeLocked(s);
        if (e != KvCacheError::None) return e;
    }
    promotions_.erase(promotion_id);
    return KvCacheError::None;
}

std::optional<PromotionTransactionSnapshot> KvCacheManager::promotionTransaction(PromotionId promotion_id) const
{
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = promotions_.find(promotion_id);
    if (it == promotions_.end()) return std::nullopt;
    Promotion const& p = it->second;
    return PromotionTransactionSnapshot{p.id, p.request_id, p.prepared_version, p.logical_token_begin, p.sources,
                                        p.target};
}

// ---- leases ---------------------------------------------------------------------------

PageLeaseAcquireResult KvCacheManager::leaseLocked(std::vector<PageHandle> handles, BlockTable table)
{
    PageLeaseAcquireResult result;
    for (PageHandle const h : handles) {
        Page const* p = page(h);
        if (p == nullptr || p->state == PageState::Free || p->state == PageState::Retiring
            || p->inflight_readers == kU32Max) {
            result.error = KvCacheError::InvalidState;
            return result;
        }
    }
    PageLeaseId const id = nextId(next_lease_id_, leases_);
    if (id == kInvalidPageLeaseId) {
        result.error = KvCacheError::InternalInvariantViolation;
        return result;
    }
    result.table = std::move(table);
    result.handles = handles;
    auto inserted = leases_.emplace(id, std::move(handles));
    if (!inserted.second) {
        result.error = KvCacheError::InternalInvariantViolation;
        return result;
    }
    for (PageHandle const h : inserted.first->second) ++page(h)->inflight_readers;
    result.error = KvCacheError::None;
    result.lease_id = id;
    return result;
}

PageLeaseAcquireResult KvCacheManager::acquireRequestReadLease(RequestId request_id)
{
    PageLeaseAcquireResult result;
    if (request_id == kInvalidRequestId) {
        result.error = KvCacheError::InvalidArgument;
        return result;
    }
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = tables_.find(request_id);
    if (it == tables_.end()) {
        result.error = KvCacheError::RequestNotFound;
        return result;
    }
    std::vector<PageHandle> handles;
    handles.reserve(it->second.entries_.size());
    for (MappingEntry const& e : it->second.entries_) handles.push_back(e.handle);
    return leaseLocked(std::move(handles), it->second);
}

PageLeaseAcquireResult KvCacheManager::acquirePromotionIoLease(PromotionId promotion_id)
{
    PageLeaseAcquireResult result;
    if (promotion_id == kInvalidPromotionId) {
        result.error = KvCacheError::InvalidArgument;
        return result;
    }
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = promotions_.find(promotion_id);
    if (it == promotions_.end()) {
        result.error = KvCacheError::PromotionNotFound;
        return result;
    }
    std::vector<PageHandle> handles(it->second.sources.begin(), it->second.sources.end());
    handles.push_back(it->second.target);
    return leaseLocked(std::move(handles), BlockTable{});
}

KvCacheError KvCacheManager::releasePageLease(PageLeaseId lease_id)
{
    if (lease_id == kInvalidPageLeaseId) return KvCacheError::InvalidArgument;
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = leases_.find(lease_id);
    if (it == leases_.end()) return KvCacheError::InvalidState;
    for (PageHandle const h : it->second) {
        Page const* p = page(h);
        if (p == nullptr || p->state == PageState::Free || p->inflight_readers == 0) {
            return KvCacheError::InternalInvariantViolation;
        }
    }
    std::vector<PageHandle> const handles = std::move(it->second);
    leases_.erase(it);
    for (PageHandle const h : handles) {
        Page* p = page(h);
        --p->inflight_readers;
        if (p->state == PageState::Retiring && p->ref_count == 0 && p->promotion_pins == 0
            && p->inflight_readers == 0) {
            KvCacheError const e = freeLocked(h);
            if (e != KvCacheError::None) return e;
        }
    }
    return KvCacheError::None;
}

// ---- inspection ------------------------------------------------------------------------

std::optional<BlockTable> KvCacheManager::blockTable(RequestId request_id) const
{
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = tables_.find(request_id);
    if (it == tables_.end()) return std::nullopt;
    return it->second;
}

std::optional<PageMetadataSnapshot> KvCacheManager::pageMetadata(PageHandle handle) const
{
    std::lock_guard<std::mutex> lock(mutex_);
    Page const* p = page(handle);
    if (p == nullptr) return std::nullopt;
    return PageMetadataSnapshot{handle, p->state, p->valid_tokens, p->ref_count, p->promotion_pins,
                                p->inflight_readers, p->mutable_owner};
}

KvCacheManagerSnapshot KvCacheManager::snapshot() const
{
    std::lock_guard<std::mutex> lock(mutex_);
    return KvCacheManagerSnapshot{tables_.size(), promotions_.size(), leases_.size(), reservations_.size(),
                                  micro_pool_.snapshot(), extent_pool_.snapshot()};
}

bool KvCacheManager::checkInvariants() const
{
    std::lock_guard<std::mutex> lock(mutex_);
    return invariantsLocked();
}

}  // namespace kimkvcache
