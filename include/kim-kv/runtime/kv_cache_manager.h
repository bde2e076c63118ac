// Heterogeneous KV page metadata manager
// (include/kim-kv/runtime/kv_cache_manager.h of the reference): multi-token
// append, single-token reservations, fork/seal/release with copy-on-write of
// shared partial tails, 8 x micro -> extent promotion and page leases.
// Every public call takes one internal mutex; errors are returned, not thrown.
#pragma once

#include "kim-kv/core/block_table.h"
#include "kim-kv/core/page_pool.h"
#include "kim-kv/core/page_state.h"
#include "kim-kv/runtime/page_lease.h"
#include "kim-kv/runtime/promotion.h"
#include "kim-kv/runtime/token_reservation.h"

#include <array>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <optional>
#include <unordered_map>
#include <vector>

namespace kimkvcache {

struct PageMetadataSnapshot final {
    PageHandle handle{PageHandle::invalid()};
    PageState state{PageState::Free};
    std::uint16_t valid_tokens{0};
    std::uint32_t ref_count{0};
    std::uint32_t promotion_pins{0};
    std::uint32_t inflight_readers{0};
    RequestId mutable_owner{kInvalidRequestId};

    [[nodiscard]] constexpr bool shared() const noexcept { return state == PageState::Sealed && ref_count > 1; }
};

struct KvCacheManagerSnapshot final {
    std::uint64_t request_count{0};
    std::uint64_t promotion_count{0};
    std::uint64_t page_lease_count{0};
    std::uint64_t token_reservation_count{0};
    PagePoolSnapshot micro_pool{};
    PagePoolSnapshot extent_pool{};
};

// A reservation of KvCacheManager::reserveTokenDelta, described by what it
// changes instead of by two full tables: the candidate table is the committed
// one (version `committed_version`, last entry `previous_tail` when
// `has_previous_tail`) with `tail` appended when `appended`, else with its last
// entry replaced by `tail`; it holds `entry_count` entries.  No counterpart in
// the reference, whose reserveToken returns both tables: this form lets a
// caller keep a device-resident copy of the table and patch one entry per
// token.
struct TokenReservationDelta final {
    KvCacheError error{KvCacheError::None};
    KvTokenReservationId reservation_id{kInvalidKvTokenReservationId};
    RequestId request_id{kInvalidRequestId};
    std::uint32_t logical_token_position{0};
    std::uint64_t committed_version{0};
    std::uint32_t entry_count{0};
    bool appended{false};
    bool has_previous_tail{false};
    MappingEntry tail{};
    MappingEntry previous_tail{};

    [[nodiscard]] constexpr bool ok() const noexcept
    {
        return error == KvCacheError::None && reservation_id != kInvalidKvTokenReservationId;
    }
};

// What KvCacheManager::appendWithLease changed: the table's entries from
// `first_entry` on (the extended or copy-on-write-replaced partial tail, then
// the fresh pages), the copy-on-write source when a shared partial tail was
// replaced, and a read lease on exactly the pages a device copy of the new
// tokens touches (those entries' pages and the replaced tail).  No
// counterpart in the reference, whose callers lease and copy the whole table
// before and after append().
struct AppendChange final {
    KvCacheError error{KvCacheError::None};
    std::uint32_t logical_token_begin{0};              // committed tokens before the append
    std::uint64_t version{0};                          // the table's new version
    std::size_t first_entry{0};
    std::vector<MappingEntry> entries;
    PageHandle replaced_tail{PageHandle::invalid()};
    std::uint16_t replaced_tokens{0};
    PageLeaseId lease_id{kInvalidPageLeaseId};

    [[nodiscard]] bool ok() const noexcept { return error == KvCacheError::None && lease_id != kInvalidPageLeaseId; }
};

class KvCacheManager final {
public:
    KvCacheManager(std::uint32_t micro_capacity, std::uint32_t extent_capacity);

    KvCacheManager(KvCacheManager const&) = delete;
    KvCacheManager& operator=(KvCacheManager const&) = delete;
    KvCacheManager(KvCacheManager&&) = delete;
    KvCacheManager& operator=(KvCacheManager&&) = delete;

    [[nodiscard]] KvCacheError createRequest(RequestId request_id);
    [[nodiscard]] KvCacheError append(RequestId request_id, std::uint32_t token_count);
    // append() in time proportional to the appended tokens (no table copy),
    // plus the lease described at AppendChange; release it with
    // releasePageLease once the device copy is done.
    [[nodiscard]] AppendChange appendWithLease(RequestId request_id, std::uint32_t token_count);

    [[nodiscard]] TokenReservationResult reserveToken(RequestId request_id,
                                                      std::uint32_t expected_committed_tokens);
    // The same reservation as reserveToken (same checks, errors, ids and page
    // staging) in O(1): no table is copied.
    [[nodiscard]] TokenReservationDelta reserveTokenDelta(RequestId request_id,
                                                          std::uint32_t expected_committed_tokens);
    [[nodiscard]] KvCacheError commitTokenReservation(KvTokenReservationId reservation_id);
    [[nodiscard]] KvCacheError rollbackTokenReservation(KvTokenReservationId reservation_id);

    [[nodiscard]] KvCacheError sealTail(RequestId request_id);
    [[nodiscard]] KvCacheError forkRequest(RequestId source_request_id, RequestId child_request_id);
    [[nodiscard]] KvCacheError releaseRequest(RequestId request_id);

    // Prepare pins metadata and lifetimes only; the caller copies the data
    // and then commits, or rolls back on any failure.
    [[nodiscard]] PromotionPrepareResult preparePromotion(RequestId request_id,
                                                          std::uint32_t logical_token_begin);
    [[nodiscard]] KvCacheError commitPromotion(PromotionId promotion_id);
    [[nodiscard]] KvCacheError rollbackPromotion(PromotionId promotion_id);

    // Snapshot of a request's table plus +1 inflight reader on every page.
    [[nodiscard]] PageLeaseAcquireResult acquireRequestReadLease(RequestId request_id);
    // Pins a prepared promotion's 8 sources and its target for the copy.
    [[nodiscard]] PageLeaseAcquireResult acquirePromotionIoLease(PromotionId promotion_id);
    // Pins a reservation's candidate pages (and a COW-replaced tail).
    [[nodiscard]] PageLeaseAcquireResult acquireTokenReservationLease(KvTokenReservationId reservation_id);
    [[nodiscard]] KvCacheError releasePageLease(PageLeaseId lease_id);

    [[nodiscard]] std::optional<BlockTable> blockTable(RequestId request_id) const;
    [[nodiscard]] std::optional<PageMetadataSnapshot> pageMetadata(PageHandle handle) const;
    [[nodiscard]] std::optional<PromotionTransactionSnapshot> promotionTransaction(PromotionId promotion_id) const;
    [[nodiscard]] KvCacheManagerSnapshot snapshot() const;
    [[nodiscard]] bool checkInvariants() const;

private:
    struct Page final {               // runtime metadata of one physical slot
        PageState state{PageState::Free};
        std::uint32_t generation{0};
        std::uint16_t valid_tokens{0};
        std::uint32_t ref_count{0};
        std::uint32_t promotion_pins{0};
        std::uint32_t inflight_readers{0};
        RequestId mutable_owner{kInvalidRequestId};
    };

    struct Promotion final {
        PromotionId id{kInvalidPromotionId};
        RequestId request_id{kInvalidRequestId};
        std::uint64_t prepared_version{0};
        std::uint32_t logical_token_begin{0};
        std::size_t first_entry{0};
        std::array<PageHandle, kPromotionSourcePageCount> sources{};
        PageHandle target{PageHandle::invalid()};
    };

    struct Reservation final {
        KvTokenReservationId id{kInvalidKvTokenReservationId};
        RequestId request_id{kInvalidRequestId};
        std::uint64_t prepared_version{0};
        MappingEntry tail{};                               // the candidate's last entry
        bool appended{false};                              // new entry, else replaces the last
        PageHandle staged{PageHandle::invalid()};          // freshly allocated tail page
        PageHandle existing_mutable{PageHandle::invalid()};
        PageHandle replaced_tail{PageHandle::invalid()};   // sealed partial tail being COW-replaced
    };

    struct Staged final {
        PageHandle handle{PageHandle::invalid()};
        std::size_t entry{0};
    };

    struct Expected;   // invariant-check accumulators

    [[nodiscard]] Page* page(PageHandle handle) noexcept;
    [[nodiscard]] Page const* page(PageHandle handle) const noexcept;
    [[nodiscard]] PagePool& pool(PageKind kind) noexcept { return kind == PageKind::Micro ? micro_pool_ : extent_pool_; }

    [[nodiscard]] KvCacheError stageMicroLocked(std::uint16_t initial_valid_tokens, PageHandle& out);
    [[nodiscard]] KvCacheError stageExtentLocked(PageHandle& out);
    void unstageLocked(std::vector<Staged> const& staged) noexcept;
    [[nodiscard]] KvCacheError dropReferenceLocked(PageHandle handle);
    [[nodiscard]] KvCacheError freeLocked(PageHandle handle);
    static void clearFreed(Page& p) noexcept;

    template <typename Map>
    [[nodiscard]] static std::uint64_t nextId(std::uint64_t& counter, Map const& live);

    [[nodiscard]] bool hasReservationLocked(RequestId request_id) const noexcept;
    // append()'s body: with `change` only the changed entries are checked and
    // the lease is taken, else the whole candidate table is checked.
    [[nodiscard]] KvCacheError appendLocked(RequestId request_id, std::uint32_t token_count, AppendChange* change);
    // reserveToken's body; with `candidate` the full candidate table is built
    // there and checked whole, else only its changed tail is checked.
    [[nodiscard]] TokenReservationDelta reserveLocked(RequestId request_id, std::uint32_t expected_committed_tokens,
                                                      BlockTable* candidate);
    [[nodiscard]] static BlockTable candidateOf(Reservation const& r, BlockTable const& committed);
    [[nodiscard]] PageLeaseAcquireResult leaseLocked(std::vector<PageHandle> handles, BlockTable table);
    [[nodiscard]] KvCacheError rollbackPromotionLocked(PromotionId promotion_id);
    [[nodiscard]] KvCacheError rollbackRequestPromotionsLocked(RequestId request_id);
    [[nodiscard]] KvCacheError rollbackReservationLocked(KvTokenReservationId reservation_id);

    [[nodiscard]] bool invariantsLocked() const;
    [[nodiscard]] bool requestInvariantsLocked(Expected& expected) const;
    [[nodiscard]] bool promotionInvariantsLocked(Expected& expected) const;
    [[nodiscard]] bool reservationInvariantsLocked(Expected& expected) const;
    [[nodiscard]] bool leaseInvariantsLocked(Expected& expected) const;
    [[nodiscard]] bool poolInvariantsLocked(PageKind kind, Expected const& expected) const;

    PagePool micro_pool_;
    PagePool extent_pool_;
    std::vector<Page> micro_pages_;
    std::vector<Page> extent_pages_;

    std::unordered_map<RequestId, BlockTable> tables_;
    std::unordered_map<PromotionId, Promotion> promotions_;
    std::unordered_map<KvTokenReservationId, Reservation> reservations_;
    std::unordered_map<RequestId, KvTokenReservationId> reservation_of_;
    std::unordered_map<PageLeaseId, std::vector<PageHandle>> leases_;

    std::uint64_t next_promotion_id_{1};
    std::uint64_t next_reservation_id_{1};
    std::uint64_t next_lease_id_{1};

    mutable std::mutex mutex_;
};

}  // namespace kimkvcache
