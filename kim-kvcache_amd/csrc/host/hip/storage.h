// HipKvStorage: the host side of the device pools (counterpart of the
// reference's src/cuda/kv/storage.h:18-166).  It owns a kimkv_storage from the
// C-ABI, validates tables against it, converts block tables to device
// descriptors and stages small per-launch uploads without blocking the host.
#pragma once

#include "kimkv_hip.h"

#include "kim-kv/core/block_table.h"
#include "kim-kv/core/kv_layout.h"
#include "kim-kv/hip/hip_status.h"
#include "kim-kv/runtime/kv_cache_manager.h"
#include "kim-kv/runtime/promotion.h"
#include "ring_regions.h"

#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <vector>

namespace kimkvcache {

HipStatus mapStatus(kimkv_status s, HipError failure) noexcept;

// Owning device allocation.
class DeviceMemory final {
public:
    DeviceMemory() = default;
    explicit DeviceMemory(std::size_t bytes);
    ~DeviceMemory();
    DeviceMemory(DeviceMemory&& o) noexcept : ptr_(o.ptr_), bytes_(o.bytes_) { o.ptr_ = nullptr; o.bytes_ = 0; }
    DeviceMemory& operator=(DeviceMemory&& o) noexcept;
    DeviceMemory(DeviceMemory const&) = delete;
    DeviceMemory& operator=(DeviceMemory const&) = delete;

    [[nodiscard]] void* get() const noexcept { return ptr_; }
    [[nodiscard]] std::size_t size() const noexcept { return bytes_; }
    [[nodiscard]] bool ok() const noexcept { return ptr_ != nullptr || bytes_ == 0; }

private:
    void* ptr_{nullptr};
    std::size_t bytes_{0};
};

// Pinned host ring (+ a device ring of the same size for upload()).  stage()
// hands kernels the pinned bytes directly; upload() / uploadTo() enqueue an
// H2D copy of them.  Every region remembers the stream whose work consumes
// it; fence(stream) records one event after that work and attaches it to all
// of the stream's unfenced regions.  A region is reused only after its event
// (or, when it was never fenced, its stream) has completed, so callers may
// fence once after several staged launches on the same stream.
class StagingRing final {
public:
    explicit StagingRing(std::size_t bytes);
    ~StagingRing();
    StagingRing(StagingRing const&) = delete;
    StagingRing& operator=(StagingRing const&) = delete;

    [[nodiscard]] bool ok() const noexcept { return host_ != nullptr && device_.get() != nullptr; }
    [[nodiscard]] std::size_t capacity() const noexcept { return size_; }
    // Largest single stage() / upload().
    [[nodiscard]] std::size_t maxStage() const noexcept { return regions_.maxRequest(); }
    // Copies `bytes` into the pinned ring and returns that host address, which
    // kernels read directly (mapped, coherent host memory: no copy command on
    // the stream).  For small per-launch argument arrays read once per
    // workgroup.  nullptr on failure.
    [[nodiscard]] void* stage(void const* data, std::size_t bytes, HipStream stream);
    // Returns the device address of the staged copy, or nullptr on failure.
    [[nodiscard]] void* upload(void const* data, std::size_t bytes, HipStream stream);
    // Device scratch of `bytes` (16-byte aligned, contents undefined) that
    // work on `stream` may use until the next fence's work completes; nullptr
    // on failure.  No copy command.
    [[nodiscard]] void* deviceScratch(std::size_t bytes, HipStream stream);
    // Host staging only (the caller names the device destination).  Any
    // size: uploads beyond half the ring are split into pieces.
    [[nodiscard]] bool uploadTo(void* device_dst, void const* data, std::size_t bytes, HipStream stream);
    void fence(HipStream stream);

private:
    struct Consumer {
        HipStream stream;   // the stream whose work consumes the region
        void* event;        // nullptr until fenced; shared by the regions one fence covered
        bool done;          // consumer known complete (stream drained)
    };
    [[nodiscard]] std::size_t reserve(std::size_t bytes, HipStream stream);
    void dropRef(void* event);

    std::size_t size_;
    unsigned char* host_{nullptr};
    unsigned char* view_{nullptr};   // device address of host_ (mapped, coherent)
    DeviceMemory device_;
    RingRegions<Consumer> regions_;
    std::vector<std::pair<void*, int>> event_refs_;   // fence events and how many live regions use each
    std::vector<void*> spare_events_;
    std::mutex mutex_;
};

// Size-class cache of device buffers (per-transaction descriptor arrays).
class DeviceBufferCache final {
public:
    ~DeviceBufferCache();
    [[nodiscard]] void* acquire(std::size_t bytes, std::size_t& granted);
    void release(void* ptr, std::size_t granted) noexcept;

private:
    std::map<std::size_t, std::vector<void*>> free_;
    std::mutex mutex_;
};

class HipKvStorage final {
public:
    HipKvStorage(KvLayout layout, std::uint32_t micro_capacity, std::uint32_t extent_capacity,
                 std::uint16_t micro_page_tokens = kMicroPageTokenCapacity,
                 std::uint16_t extent_page_tokens = kExtentPageTokenCapacity) noexcept;
    ~HipKvStorage();
    HipKvStorage(HipKvStorage const&) = delete;
    HipKvStorage& operator=(HipKvStorage const&) = delete;

    [[nodiscard]] HipStatus status() const noexcept { return status_; }
    [[nodiscard]] kimkv_storage* handle() const noexcept { return storage_; }
    [[nodiscard]] KvLayout layout() const noexcept { return layout_; }
    [[nodiscard]] HipStorageSnapshot snapshot() const noexcept;
    [[nodiscard]] std::uint16_t pageTokenCapacity(PageKind kind) const noexcept
    {
        return kind == PageKind::Micro ? micro_tokens_ : extent_tokens_;
    }
    [[nodiscard]] bool pageExists(PageHandle handle) const noexcept;
    // Structure (standard or uniform capacities) plus every page in range
    // (CudaKvStorage::Impl::validTable, src/cuda/kv/storage.cpp:79-97).  For
    // the standard 8/64 layout the distinct-page check is a stamp per pool
    // slot, linear in the entry count (a reserve at 32k tokens checks ~514
    // entries twice per lane per token).
    [[nodiscard]] bool validTable(BlockTable const& table) const;
    void descriptors(BlockTable const& table, std::vector<kimkv_block_desc>& out) const;
    // One entry's descriptor; false when its page is out of range, its kind
    // disagrees with its handle or its token count with the page capacity.
    [[nodiscard]] bool descriptor(MappingEntry const& entry, kimkv_block_desc& out) const noexcept;

    [[nodiscard]] bool consumeFailure(HipFailurePoint point) noexcept;
    void injectFailureOnce(HipFailurePoint point) noexcept;

    StagingRing& ring() noexcept { return ring_; }
    // Held around every staged upload + launch + fence on this storage, so a
    // fence always covers the regions staged just before it.
    std::mutex& launchMutex() noexcept { return launch_mutex_; }
    DeviceBufferCache& buffers() noexcept { return buffers_; }
    // Device block-table writes enqueued on this storage so far (reserve
    // patches, prefill table uploads), counted under launchMutex(): data
    // derived from the tables' device contents is reusable while it holds.
    void noteDescriptorWrite() noexcept { ++descriptor_writes_; }
    [[nodiscard]] std::uint64_t descriptorWrites() const noexcept { return descriptor_writes_; }

    // Synchronous data-path operations used by HipKvCache: enqueue on
    // `stream`, then wait for completion.
    [[nodiscard]] HipStatus append(BlockTable const& before, BlockTable const& after,
                                   std::uint32_t append_token_begin, std::uint32_t token_count,
                                   KvScalar const* device_input, HipStream stream);
    // Jobs of one metadata append from its AppendChange (the new tokens land
    // in change.entries; the first of them continues the copy-on-write
    // source, if any) for a [layer][K/V][count][head][dim] input.  Checks
    // every named page and the copy-on-write rule; false leaves `jobs` as it
    // was.  Proportional to the appended tokens, not to the table.
    [[nodiscard]] bool changeJobs(AppendChange const& change, std::uint32_t count, KvScalar const* input,
                                  std::vector<kimkv_append_job>& jobs) const;
    // One launch of jobs from changeJobs (several requests), waited for.
    [[nodiscard]] HipStatus appendJobsNow(std::vector<kimkv_append_job> const& jobs, HipStream stream);
    [[nodiscard]] HipStatus gather(BlockTable const& table, KvScalar* device_output, HipStream stream);
    [[nodiscard]] HipStatus promote(PromotionPrepareResult const& promotion, HipStream stream);
    [[nodiscard]] HipStatus promoteBatch(std::vector<PromotionPrepareResult> const& promotions, HipStream stream);
    [[nodiscard]] HipStatus referenceAttention(BlockTable const& table, float const* device_query,
                                               float* device_output, HipStream stream);

private:
    [[nodiscard]] HipStatus finish(HipStream stream, HipStatus submitted) noexcept;
public:
    // Segments of one request's append [begin, begin + count): one job per
    // touched entry with destination, token count and copy-on-write source
    // filled in (validates both tables and the COW rule); token_offsets gets
    // each job's first token relative to `begin`.  Sources are left to the
    // caller.
    [[nodiscard]] bool appendSegments(BlockTable const& before, BlockTable const& after, std::uint32_t begin,
                                      std::uint32_t count, std::vector<kimkv_append_job>& jobs,
                                      std::vector<std::uint32_t>& token_offsets) const;

private:
    // Jobs of one request's append from a [layer][K/V][count][head][dim] input.
    [[nodiscard]] bool appendJobs(BlockTable const& before, BlockTable const& after, std::uint32_t begin,
                                  std::uint32_t count, KvScalar const* input,
                                  std::vector<kimkv_append_job>& jobs) const;
    [[nodiscard]] HipStatus launchAppendJobs(std::vector<kimkv_append_job> const& jobs, HipStream stream);

    KvLayout layout_{};
    std::uint32_t micro_capacity_{0};
    std::uint32_t extent_capacity_{0};
    std::uint16_t micro_tokens_{0};
    std::uint16_t extent_tokens_{0};
    kimkv_storage* storage_{nullptr};
    HipStatus status_{};
    StagingRing ring_;
    std::mutex launch_mutex_;
    std::uint64_t descriptor_writes_{0};
    DeviceBufferCache buffers_;
    // Per-slot visit stamps for the O(entries) duplicate-page check.
    mutable std::mutex stamp_mutex_;
    mutable std::vector<std::uint32_t> micro_stamp_;
    mutable std::vector<std::uint32_t> extent_stamp_;
    mutable std::uint32_t stamp_{0};
    std::mutex fault_mutex_;
    bool fail_submission_once_{false};
    bool fail_completion_once_{false};
};

}  // namespace kimkvcache
