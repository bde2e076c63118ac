// HipKvCache: metadata + device pools for the micro-benchmark path
// (semantics of src/cuda/kv/cache.cpp:76-293 in the reference: read leases
// around every device access, a failed device append cancels the request,
// a failed promotion copy rolls the promotion back).  An append leases only
// the pages its copy touches and builds its jobs from the manager's change
// record, so its cost does not grow with the context (the reference leases
// and copies the whole table before and after).
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
    HipKvOperationResult result;
    appendBatch(&request_id, 1, token_count, &device_input, stream, &result);
    if (result.ok() && !manager_.blockTable(request_id).has_value()) {
        return metadataFailure(KvCacheError::RequestNotFound);
    }
    return result;
}

// Per request: the manager's in-place append, which also leases exactly the
// pages the copy touches (the new tokens' pages and a copy-on-write source),
// and that change's jobs; then one append launch for every request, waited
// for, and the leases released.  A request whose pages do not check out, or
// every request of a failed launch, is cancelled: its metadata append is
// committed but its pages are not written.
void HipKvCache::appendBatch(RequestId const* request_ids, std::size_t count, std::uint32_t token_count,
                             KvScalar const* const* device_inputs, HipStream stream, HipKvOperationResult* results)
{
    struct Pending {
        std::size_t index;
        PageLeaseId lease;
    };
    thread_local std::vector<Pending> pending;
    thread_local std::vector<kimkv_append_job> jobs;
    pending.clear();
    jobs.clear();
    HipStatus const st = status();
    auto settle = [&](std::size_t i, PageLeaseId lease, HipStatus device) {
        KvCacheError const l = manager_.releasePageLease(lease);
        if (!device.ok()) {
            KvCacheError const c = manager_.releaseRequest(request_ids[i]);
            results[i] = HipKvOperationResult{
                c != KvCacheError::None && c != KvCacheError::RequestNotFound ? c : KvCacheError::None, device};
        } else {
            results[i] = l == KvCacheError::None ? HipKvOperationResult{} : metadataFailure(l);
        }
    };
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
        AppendChange const change = manager_.appendWithLease(id, token_count);
        if (!change.ok()) {
            results[i] = metadataFailure(change.error);
            continue;
        }
        if (!storage_->changeJobs(change, token_count, device_inputs[i], jobs)) {
            settle(i, change.lease_id, HipStatus{HipError::InvalidArgument, 0});
            continue;
        }
        pending.push_back(Pending{i, change.lease_id});
    }
    if (pending.empty()) return;
    HipStatus const device = storage_->appendJobsNow(jobs, stream);
    for (Pending const& p : pending) settle(p.index, p.lease, device);
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
