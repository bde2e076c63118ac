// HipKvCache: metadata + device pools for the micro-benchmark path
// (semantics of src/cuda/kv/cache.cpp:76-293 in the reference: read leases
// around every device access, a failed device append cancels the request,
// a failed promotion copy rolls the promotion back).
#include "kim-kv/hip/hip_kv_cache.h"

#include "storage.h"

#include <vector>

namespace kimkvcache {
namespace {

HipKvOperationResult metadataFailure(KvCacheError e) noexcept { return HipKvOperationResult{e, HipStatus{}}; }

}  // namespace

HipKvCache::HipKvCache(KvLayout layout, std::uint32_t micro_capacity, std::uint32_t extent_capacity)
    : manager_(micro_capacity, extent_capacity),
      storage_(std::make_unique<HipKvStorage>(layout, micro_capacity, extent_capacity))
{
}

HipKvCache::~HipKvCache() = default;

HipStatus HipKvCache::status() const noexcept
{
    return storage_ != nullptr ? storage_->status() : HipStatus{HipError::AllocationFailed, 0};
}

void const* HipKvCache::storageHandle() const noexcept { return storage_ != nullptr ? storage_->handle() : nullptr; }

KvCacheError HipKvCache::createRequest(RequestId id) { return manager_.createRequest(id); }
KvCacheError HipKvCache::sealTail(RequestId id) { return manager_.sealTail(id); }
KvCacheError HipKvCache::forkRequest(RequestId s, RequestId c) { return manager_.forkRequest(s, c); }
KvCacheError HipKvCache::releaseRequest(RequestId id) { return manager_.releaseRequest(id); }

HipKvOperationResult HipKvCache::append(RequestId request_id, std::uint32_t token_count, KvScalar const* device_input,
                                        HipStream stream)
{
    if (request_id == kInvalidRequestId || token_count == 0 || device_input == nullptr) {
        return metadataFailure(KvCacheError::InvalidArgument);
    }
    HipStatus const st = status();
    if (!st.ok()) return HipKvOperationResult{KvCacheError::None, st};
    PageLeaseAcquireResult before = manager_.acquireRequestReadLease(request_id);
    if (!before.ok()) return metadataFailure(before.error);
    std::uint32_t const begin = before.table.tokenCount();
    KvCacheError const appended = manager_.append(request_id, token_count);
    if (appended != KvCacheError::None) {
        KvCacheError const l = manager_.releasePageLease(before.lease_id);
        return metadataFailure(l == KvCacheError::None ? appended : l);
    }
    PageLeaseAcquireResult after = manager_.acquireRequestReadLease(request_id);
    if (!after.ok()) {
        KvCacheError const l = manager_.releasePageLease(before.lease_id);
        if (after.error != KvCacheError::RequestNotFound) static_cast<void>(manager_.releaseRequest(request_id));
        return metadataFailure(l == KvCacheError::None ? after.error : l);
    }
    HipStatus const device = storage_->append(before.table, after.table, begin, token_count, device_input, stream);
    KvCacheError const ra = manager_.releasePageLease(after.lease_id);
    KvCacheError const rb = manager_.releasePageLease(before.lease_id);
    if (ra != KvCacheError::None) return metadataFailure(ra);
    if (rb != KvCacheError::None) return metadataFailure(rb);
    if (!device.ok()) {
        // The metadata append is committed but the pages are not: cancel the
        // request rather than expose uninitialised KV.
        KvCacheError const c = manager_.releaseRequest(request_id);
        if (c != KvCacheError::None && c != KvCacheError::RequestNotFound) return HipKvOperationResult{c, device};
        return HipKvOperationResult{KvCacheError::None, device};
    }
    if (!manager_.blockTable(request_id).has_value()) return metadataFailure(KvCacheError::RequestNotFound);
    return {};
}

void HipKvCache::appendBatch(RequestId const* request_ids, std::size_t count, std::uint32_t token_count,
                             KvScalar const* const* device_inputs, HipStream stream, HipKvOperationResult* results)
{
    struct Pending {
        std::size_t index;
        PageLeaseAcquireResult before;
        PageLeaseAcquireResult after;
        std::uint32_t begin;
    };
    std::vector<Pending> pending;
    pending.reserve(count);
    HipStatus const st = status();
    for (std::size_t i = 0; i < count; ++i) {
        RequestId const id = request_ids[i];
        if (id == kInvalidRequestId || token_count == 0 || device_inputs[i] == nullptr) {
            results[i] = metadataFailure(KvCacheError::InvalidArgument);
            continue;
        }
        if (!st.ok()) {
            results[i] = HipKvOperationResult{KvCacheError::None, st};
            continue;
        }
        PageLeaseAcquireResult before = manager_.acquireRequestReadLease(id);
        if (!before.ok()) {
            results[i] = metadataFailure(before.error);
            continue;
        }
        std::uint32_t const begin = before.table.tokenCount();
        KvCacheError const appended = manager_.append(id, token_count);
        if (appended != KvCacheError::None) {
            KvCacheError const l = manager_.releasePageLease(before.lease_id);
            results[i] = metadataFailure(l == KvCacheError::None ? appended : l);
            continue;
        }
        PageLeaseAcquireResult after = manager_.acquireRequestReadLease(id);
        if (!after.ok()) {
            KvCacheError const l = manager_.releasePageLease(before.lease_id);
            if (after.error != KvCacheError::RequestNotFound) static_cast<void>(manager_.releaseRequest(id));
            results[i] = metadataFailure(l == KvCacheError::None ? after.error : l);
            continue;
        }
        pending.push_back(Pending{i, std::move(before), std::move(after), begin});
    }
    if (pending.empty()) return;
    std::vector<HipKvStorage::AppendPlan> plans;
    plans.reserve(pending.size());
    for (Pending const& p : pending) {
        plans.push_back(HipKvStorage::AppendPlan{&p.before.table, &p.after.table, p.begin, token_count,
                                                 device_inputs[p.index]});
    }
    HipStatus const device = storage_->appendMany(plans, stream);
    for (Pending& p : pending) {
        KvCacheError const ra = manager_.releasePageLease(p.after.lease_id);
        KvCacheError const rb = manager_.releasePageLease(p.before.lease_id);
        RequestId const id = request_ids[p.index];
        if (!device.ok()) {
            KvCacheError const c = manager_.releaseRequest(id);
            results[p.index] = HipKvOperationResult{
                c != KvCacheError::None && c != KvCacheError::RequestNotFound ? c : KvCacheError::None, device};
            continue;
        }
        if (ra != KvCacheError::None) {
            results[p.index] = metadataFailure(ra);
        } else if (rb != KvCacheError::None) {
            results[p.index] = metadataFailure(rb);
        } else {
            results[p.index] = {};
        }
    }
}

HipKvOperationResult HipKvCache::promote(RequestId request_id, std::uint32_t logical_token_begin, HipStream stream)
{
    HipStatus const st = status();
    if (!st.ok()) return HipKvOperationResult{KvCacheError::None, st};
    PromotionPrepareResult const p = manager_.preparePromotion(request_id, logical_token_begin);
    if (!p.ok()) return metadataFailure(p.error);
    PageLeaseAcquireResult lease = manager_.acquirePromotionIoLease(p.promotion_id);
    if (!lease.ok()) {
        KvCacheError const r = manager_.rollbackPromotion(p.promotion_id);
        return metadataFailure(r == KvCacheError::None ? lease.error : r);
    }
    HipStatus const device = storage_->promote(p, stream);
    KvCacheError const l = manager_.releasePageLease(lease.lease_id);
    if (l != KvCacheError::None) {
        static_cast<void>(manager_.rollbackPromotion(p.promotion_id));
        return metadataFailure(l);
    }
    if (!device.ok()) {
        KvCacheError const r = manager_.rollbackPromotion(p.promotion_id);
        if (r != KvCacheError::None && r != KvCacheError::PromotionNotFound) return HipKvOperationResult{r, device};
        return HipKvOperationResult{KvCacheError::None, device};
    }
    return HipKvOperationResult{manager_.commitPromotion(p.promotion_id), device};
}

namespace {

template <typename Op>
HipKvOperationResult leasedRead(KvCacheManager& m, RequestId id, Op op)
{
    PageLeaseAcquireResult lease = m.acquireRequestReadLease(id);
    if (!lease.ok()) return metadataFailure(lease.error);
    HipStatus const device = op(lease.table);
    KvCacheError const l = m.releasePageLease(lease.lease_id);
    if (l != KvCacheError::None) return HipKvOperationResult{l, device};
    return HipKvOperationResult{KvCacheError::None, device};
}

}  // namespace

HipKvOperationResult HipKvCache::gather(RequestId request_id, KvScalar* device_output, HipStream stream)
{
    if (request_id == kInvalidRequestId || device_output == nullptr) return metadataFailure(KvCacheError::InvalidArgument);
    HipStatus const st = status();
    if (!st.ok()) return HipKvOperationResult{KvCacheError::None, st};
    return leasedRead(manager_, request_id,
                      [&](BlockTable const& t) { return storage_->gather(t, device_output, stream); });
}

HipKvOperationResult HipKvCache::referenceAttention(RequestId request_id, float const* device_query,
                                                    float* device_output, HipStream stream)
{
    if (request_id == kInvalidRequestId || device_query == nullptr || device_output == nullptr) {
        return metadataFailure(KvCacheError::InvalidArgument);
    }
    HipStatus const st = status();
    if (!st.ok()) return HipKvOperationResult{KvCacheError::None, st};
    return leasedRead(manager_, request_id, [&](BlockTable const& t) {
        return storage_->referenceAttention(t, device_query, device_output, stream);
    });
}

std::optional<BlockTable> HipKvCache::blockTable(RequestId id) const { return manager_.blockTable(id); }
KvCacheManagerSnapshot HipKvCache::metadataSnapshot() const { return manager_.snapshot(); }
HipStorageSnapshot HipKvCache::storageSnapshot() const noexcept
{
    return storage_ != nullptr ? storage_->snapshot() : HipStorageSnapshot{};
}
bool HipKvCache::checkInvariants() const { return manager_.checkInvariants(); }
void HipKvCache::injectFailureOnce(HipFailurePoint point) noexcept
{
    if (storage_ != nullptr) storage_->injectFailureOnce(point);
}

}  // namespace kimkvcache
