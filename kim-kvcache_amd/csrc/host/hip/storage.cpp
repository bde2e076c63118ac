// HipKvStorage and its staging helpers.  Data-path behaviour follows the
// reference's CudaKvStorage (src/cuda/kv/append.cpp:10-140, gather.cpp:9-107,
// promotion.cpp:8-64, src/cuda/attention/reference_attention.cpp:10-170): the
// only old mapping whose page may change in an append is the partial micro
// tail (copy-on-write), every appended segment lands in its page at
// (segment begin - entry begin), promotions copy 8 micro pages to one extent.
#include "storage.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <new>

namespace kimkvcache {

HipStatus mapStatus(kimkv_status s, HipError failure) noexcept
{
    if (s == KIMKV_OK) return {};
    switch (s) {
    case KIMKV_INVALID_ARGUMENT: return {HipError::InvalidArgument, kimkv_last_native_error()};
    case KIMKV_RUNTIME_UNAVAILABLE: return {HipError::RuntimeUnavailable, kimkv_last_native_error()};
    case KIMKV_ALLOCATION_FAILED: return {HipError::AllocationFailed, kimkv_last_native_error()};
    case KIMKV_NOT_READY: return {HipError::NotReady, 0};
    default: return {failure, kimkv_last_native_error()};
    }
}

// ---- DeviceMemory -------------------------------------------------------------

DeviceMemory::DeviceMemory(std::size_t bytes) : bytes_(bytes)
{
    if (bytes != 0 && kimkv_device_malloc(&ptr_, bytes) != KIMKV_OK) {
        ptr_ = nullptr;
    }
}

DeviceMemory::~DeviceMemory()
{
    if (ptr_ != nullptr) static_cast<void>(kimkv_device_free(ptr_));
}

DeviceMemory& DeviceMemory::operator=(DeviceMemory&& o) noexcept
{
    if (this != &o) {
        if (ptr_ != nullptr) static_cast<void>(kimkv_device_free(ptr_));
        ptr_ = o.ptr_;
        bytes_ = o.bytes_;
        o.ptr_ = nullptr;
        o.bytes_ = 0;
    }
    return *this;
}

// ---- StagingRing -----------------------------------------------------------------

StagingRing::StagingRing(std::size_t bytes) : size_(bytes), device_(), regions_(bytes)
{
    void* host = nullptr;
    void* view = nullptr;
    if (kimkv_host_malloc_mapped(&host, &view, bytes) == KIMKV_OK) {
        host_ = static_cast<unsigned char*>(host);
        view_ = static_cast<unsigned char*>(view);
    }
}

StagingRing::~StagingRing()
{
    for (auto const& r : regions_.live()) {
        if (r.tag.done) continue;
        if (r.tag.event != nullptr) {
            static_cast<void>(kimkv_event_synchronize(r.tag.event));
        } else {
            static_cast<void>(kimkv_stream_synchronize(r.tag.stream));
        }
    }
    for (auto const& e : event_refs_) static_cast<void>(kimkv_event_destroy(e.first));
    for (void* e : spare_events_) static_cast<void>(kimkv_event_destroy(e));
    if (host_ != nullptr) static_cast<void>(kimkv_host_free_pinned(host_));
}

void StagingRing::dropRef(void* event)
{
    if (event == nullptr) return;
    auto it = std::find_if(event_refs_.begin(), event_refs_.end(),
                           [event](std::pair<void*, int> const& e) { return e.first == event; });
    if (it == event_refs_.end()) return;
    if (--it->second == 0) {
        spare_events_.push_back(event);
        event_refs_.erase(it);
    }
}

std::size_t StagingRing::reserve(std::size_t bytes, HipStream stream)
{
    // A region is free again once its own fence event has completed or, if
    // it was never fenced, once its stream has drained.
    return regions_.reserve(bytes, Consumer{stream, nullptr, false}, [this](auto const& r) {
        if (!r.tag.done) {
            if (r.tag.event != nullptr) {
                static_cast<void>(kimkv_event_synchronize(r.tag.event));
            } else {
                static_cast<void>(kimkv_stream_synchronize(r.tag.stream));
            }
        }
        dropRef(r.tag.event);
    });
}

void* StagingRing::stage(void const* data, std::size_t bytes, HipStream stream)
{
    std::lock_guard<std::mutex> lock(mutex_);
    if (host_ == nullptr || view_ == nullptr || bytes > regions_.maxRequest()) return nullptr;
    std::size_t const off = reserve(bytes, stream);
    std::memcpy(host_ + off, data, bytes);
    return view_ + off;
}

void* StagingRing::upload(void const* data, std::size_t bytes, HipStream stream)
{
    std::lock_guard<std::mutex> lock(mutex_);
    if (host_ == nullptr || bytes > regions_.maxRequest()) return nullptr;
    if (device_.get() == nullptr) device_ = DeviceMemory(size_);
    if (device_.get() == nullptr) return nullptr;
    std::size_t const off = reserve(bytes, stream);
    std::memcpy(host_ + off, data, bytes);
    unsigned char* dev = static_cast<unsigned char*>(device_.get()) + off;
    if (kimkv_memcpy_h2d_async(dev, host_ + off, bytes, stream) != KIMKV_OK) return nullptr;
    return dev;
}

void* StagingRing::deviceScratch(std::size_t bytes, HipStream stream)
{
    std::lock_guard<std::mutex> lock(mutex_);
    if (host_ == nullptr || bytes > regions_.maxRequest()) return nullptr;
    if (device_.get() == nullptr) device_ = DeviceMemory(size_);
    if (device_.get() == nullptr) return nullptr;
    std::size_t const off = reserve(bytes, stream);
    return static_cast<unsigned char*>(device_.get()) + off;
}

bool StagingRing::uploadTo(void* device_dst, void const* data, std::size_t bytes, HipStream stream)
{
    std::lock_guard<std::mutex> lock(mutex_);
    if (host_ == nullptr) return false;
    // An upload larger than one ring request goes in pieces; a piece that
    // needs the ring space of an earlier one waits for that copy (its region
    // is unfenced, so reserve drains the stream first).
    auto const* src = static_cast<unsigned char const*>(data);
    auto* dst = static_cast<unsigned char*>(device_dst);
    std::size_t const piece = regions_.maxRequest();
    for (std::size_t done = 0; done < bytes;) {
        std::size_t const n = std::min(piece, bytes - done);
        std::size_t const off = reserve(n, stream);
        std::memcpy(host_ + off, src + done, n);
        if (kimkv_memcpy_h2d_async(dst + done, host_ + off, n, stream) != KIMKV_OK) return false;
        done += n;
    }
    return true;
}

void StagingRing::fence(HipStream stream)
{
    std::lock_guard<std::mutex> lock(mutex_);
    auto unfenced = [stream](Consumer const& c) { return !c.done && c.event == nullptr && c.stream == stream; };
    int pending = 0;
    for (auto const& r : regions_.live()) pending += unfenced(r.tag) ? 1 : 0;
    if (pending == 0) return;
    void* event = nullptr;
    if (!spare_events_.empty()) {
        event = spare_events_.back();
        spare_events_.pop_back();
    } else if (kimkv_event_create(&event, KIMKV_EVENT_ORDER_ONLY) != KIMKV_OK) {
        event = nullptr;
    }
    if (event != nullptr && kimkv_event_record(event, stream) != KIMKV_OK) {
        spare_events_.push_back(event);
        event = nullptr;
    }
    if (event == nullptr) {
        // Cannot fence: drain the stream so its staged regions are free again.
        static_cast<void>(kimkv_stream_synchronize(stream));
        for (auto& r : regions_.live()) {
            if (unfenced(r.tag)) r.tag.done = true;
        }
        return;
    }
    // One event, recorded after everything staged on this stream so far,
    // covers all of that stream's unfenced regions.
    for (auto& r : regions_.live()) {
        if (unfenced(r.tag)) r.tag.event = event;
    }
    event_refs_.emplace_back(event, pending);
}

// ---- DeviceBufferCache ----------------------------------------------------------------

DeviceBufferCache::~DeviceBufferCache()
{
    for (auto& [size, list] : free_) {
        for (void* p : list) static_cast<void>(kimkv_device_free(p));
    }
}

void* DeviceBufferCache::acquire(std::size_t bytes, std::size_t& granted)
{
    std::size_t cls = 4096;
    while (cls < bytes) cls <<= 1;
    {
        std::lock_guard<std::mutex> lock(mutex_);
        auto it = free_.find(cls);
        if (it != free_.end() && !it->second.empty()) {
            void* p = it->second.back();
            it->second.pop_back();
            granted = cls;
            return p;
        }
    }
    void* p = nullptr;
    if (kimkv_device_malloc(&p, cls) != KIMKV_OK) return nullptr;
    granted = cls;
    return p;
}

void DeviceBufferCache::release(void* ptr, std::size_t granted) noexcept
{
    if (ptr == nullptr) return;
    std::lock_guard<std::mutex> lock(mutex_);
    try {
        free_[granted].push_back(ptr);
    } catch (...) {
        static_cast<void>(kimkv_device_free(ptr));
    }
}

// ---- HipKvStorage --------------------------------------------------------------------

// 8 MiB by default; KIMKV_STAGING_RING_BYTES overrides it (at least 64 KiB),
// which tests use to drive uploads through the split and wrap paths.
static std::size_t stagingRingBytes() noexcept
{
    std::size_t bytes = std::size_t{8} << 20;
    if (char const* env = std::getenv("KIMKV_STAGING_RING_BYTES")) {
        char* end = nullptr;
        unsigned long long const v = std::strtoull(env, &end, 10);
        if (end != env && *end == '\0') bytes = std::max<std::size_t>(std::size_t{64} << 10, v);
    }
    return bytes;
}

HipKvStorage::HipKvStorage(KvLayout layout, std::uint32_t micro_capacity, std::uint32_t extent_capacity,
                           std::uint16_t micro_page_tokens, std::uint16_t extent_page_tokens) noexcept
    : layout_(layout),
      micro_capacity_(micro_capacity),
      extent_capacity_(extent_capacity),
      micro_tokens_(micro_page_tokens),
      extent_tokens_(extent_page_tokens),
      ring_(stagingRingBytes())
{
    if (!layout.valid() || micro_page_tokens == 0 || extent_page_tokens == 0) {
        status_ = HipStatus{HipError::InvalidArgument, 0};
        return;
    }
    if (kimkv_device_count() == 0) {
        status_ = HipStatus{HipError::RuntimeUnavailable, 0};
        return;
    }
    kimkv_layout const l{layout.layer_count, layout.kv_head_count, layout.head_dimension};
    status_ = mapStatus(kimkv_storage_create(&storage_, l, micro_capacity, extent_capacity, micro_page_tokens,
                                             extent_page_tokens),
                        HipError::AllocationFailed);
}

HipKvStorage::~HipKvStorage()
{
    if (storage_ != nullptr) static_cast<void>(kimkv_storage_destroy(storage_));
}

HipStorageSnapshot HipKvStorage::snapshot() const noexcept
{
    HipStorageSnapshot s;
    s.micro_capacity = micro_capacity_;
    s.extent_capacity = extent_capacity_;
    s.micro_page_tokens = micro_tokens_;
    s.extent_page_tokens = extent_tokens_;
    std::size_t per_token = 0;
    if (layout_.bytesForTokens(1, per_token)) {
        s.micro_reserved_bytes = per_token * micro_tokens_ * micro_capacity_;
        s.extent_reserved_bytes = per_token * extent_tokens_ * extent_capacity_;
    }
    return s;
}

bool HipKvStorage::pageExists(PageHandle h) const noexcept
{
    if (!h.isStructurallyValid() || storage_ == nullptr) return false;
    return h.kind == PageKind::Micro ? h.slot < micro_capacity_ : h.slot < extent_capacity_;
}

bool HipKvStorage::validTable(BlockTable const& table) const
{
    bool const standard = micro_tokens_ == kMicroPageTokenCapacity && extent_tokens_ == kExtentPageTokenCapacity;
    if (!standard) {
        return extent_capacity_ == 0 && table.checkInvariants(micro_tokens_)
            && std::all_of(table.entries().begin(), table.entries().end(),
                           [this](MappingEntry const& e) { return pageExists(e.handle); });
    }
    std::uint64_t next = 0;
    for (MappingEntry const& e : table.entries()) {
        if (!pageExists(e.handle) || e.kind != e.handle.kind) return false;
        std::uint16_t const cap = pageTokenCapacity(e.kind);
        if (e.valid_tokens == 0 || e.valid_tokens > cap || e.logical_token_begin != next) return false;
        next += e.valid_tokens;
        if (next > 0xFFFFFFFFull) return false;
    }
    // No page twice: stamp each slot with this call's number.
    std::lock_guard<std::mutex> lock(stamp_mutex_);
    if (micro_stamp_.size() != micro_capacity_) micro_stamp_.assign(micro_capacity_, 0);
    if (extent_stamp_.size() != extent_capacity_) extent_stamp_.assign(extent_capacity_, 0);
    if (++stamp_ == 0) {
        std::fill(micro_stamp_.begin(), micro_stamp_.end(), 0);
        std::fill(extent_stamp_.begin(), extent_stamp_.end(), 0);
        stamp_ = 1;
    }
    for (MappingEntry const& e : table.entries()) {
        std::uint32_t& seen = (e.kind == PageKind::Micro ? micro_stamp_ : extent_stamp_)[e.handle.slot];
        if (seen == stamp_) return false;
        seen = stamp_;
    }
    return true;
}

namespace {

kimkv_block_desc toDescriptor(MappingEntry const& e, std::uint16_t capacity) noexcept
{
    kimkv_block_desc d{};
    d.slot = e.handle.slot;
    d.generation = e.handle.generation;
    d.logical_token_begin = e.logical_token_begin;
    d.valid_tokens = e.valid_tokens;
    d.page_token_capacity = capacity;
    d.kind = static_cast<std::uint8_t>(e.kind);
    return d;
}

}  // namespace

void HipKvStorage::descriptors(BlockTable const& table, std::vector<kimkv_block_desc>& out) const
{
    out.clear();
    out.reserve(table.entries().size());
    for (MappingEntry const& e : table.entries()) out.push_back(toDescriptor(e, pageTokenCapacity(e.kind)));
}

bool HipKvStorage::descriptor(MappingEntry const& entry, kimkv_block_desc& out) const noexcept
{
    if (!pageExists(entry.handle) || entry.kind != entry.handle.kind) return false;
    std::uint16_t const cap = pageTokenCapacity(entry.kind);
    if (entry.valid_tokens == 0 || entry.valid_tokens > cap) return false;
    out = toDescriptor(entry, cap);
    return true;
}

bool HipKvStorage::consumeFailure(HipFailurePoint point) noexcept
{
    std::lock_guard<std::mutex> lock(fault_mutex_);
    bool& flag = point == HipFailurePoint::Submission ? fail_submission_once_ : fail_completion_once_;
    bool const fire = flag;
    flag = false;
    return fire;
}

void HipKvStorage::injectFailureOnce(HipFailurePoint point) noexcept
{
    std::lock_guard<std::mutex> lock(fault_mutex_);
    (point == HipFailurePoint::Submission ? fail_submission_once_ : fail_completion_once_) = true;
}

HipStatus HipKvStorage::finish(HipStream stream, HipStatus submitted) noexcept
{
    kimkv_status const s = kimkv_stream_synchronize(stream);
    if (!submitted.ok()) return submitted;
    if (s != KIMKV_OK) return HipStatus{HipError::ExecutionFailed, kimkv_last_native_error()};
    if (consumeFailure(HipFailurePoint::Completion)) return HipStatus{HipError::ExecutionFailed, -1};
    return {};
}

namespace {

struct TempDevice {
    DeviceMemory mem;
    bool upload(void const* data, std::size_t bytes, HipStream stream)
    {
        mem = DeviceMemory(bytes);
        return mem.get() != nullptr && kimkv_memcpy_h2d_async(mem.get(), data, bytes, stream) == KIMKV_OK;
    }
};

}  // namespace

bool HipKvStorage::appendSegments(BlockTable const& before, BlockTable const& after, std::uint32_t begin,
                                  std::uint32_t count, std::vector<kimkv_append_job>& jobs,
                                  std::vector<std::uint32_t>& token_offsets) const
{
    std::uint64_t const end = static_cast<std::uint64_t>(begin) + count;
    if (count == 0 || end > 0xFFFFFFFFull || !validTable(before) || !validTable(after)
        || before.tokenCount() != begin || after.tokenCount() != end) {
        return false;
    }
    // Copy-on-write source of the replaced partial tail, if any.  Both
    // tables are contiguous from token 0 and `after` extends `before`, so an
    // entry of `before` can only reappear at its own index.
    PageHandle cow_src = PageHandle::invalid();
    std::uint16_t cow_tokens = 0;
    PageHandle cow_dst = PageHandle::invalid();
    if (after.entries().size() < before.entries().size()) return false;
    for (std::size_t k = 0; k < before.entries().size(); ++k) {
        MappingEntry const& old = before.entries()[k];
        auto const rep = after.entries().begin() + static_cast<std::ptrdiff_t>(k);
        if (rep->logical_token_begin != old.logical_token_begin) return false;
        if (rep->handle == old.handle) continue;
        bool const tail = old.logicalTokenEnd() == begin;
        if (!tail || old.kind != PageKind::Micro || rep->kind != PageKind::Micro || old.valid_tokens >= micro_tokens_
            || rep->valid_tokens < old.valid_tokens) {
            return false;
        }
        cow_src = old.handle;
        cow_tokens = old.valid_tokens;
        cow_dst = rep->handle;
    }
    std::size_t const first = jobs.size();
    for (MappingEntry const& e : after.entries()) {
        std::uint32_t const sb = std::max(begin, e.logical_token_begin);
        std::uint32_t const se = std::min(static_cast<std::uint32_t>(end), e.logicalTokenEnd());
        if (sb >= se) continue;
        kimkv_append_job j{};
        j.token_count = se - sb;
        token_offsets.push_back(sb - begin);
        j.dst_slot = e.handle.slot;
        j.dst_kind = static_cast<std::uint8_t>(e.kind);
        j.dst_token = static_cast<std::uint16_t>(sb - e.logical_token_begin);
        if (cow_dst.isStructurallyValid() && e.handle == cow_dst) {
            j.cow_slot = cow_src.slot;
            j.cow_kind = static_cast<std::uint8_t>(cow_src.kind);
            j.cow_tokens = cow_tokens;
        }
        jobs.push_back(j);
    }
    return jobs.size() > first;
}

bool HipKvStorage::appendJobs(BlockTable const& before, BlockTable const& after, std::uint32_t begin,
                              std::uint32_t count, KvScalar const* input, std::vector<kimkv_append_job>& jobs) const
{
    if (input == nullptr) return false;
    std::size_t const first = jobs.size();
    std::vector<std::uint32_t> offsets;
    if (!appendSegments(before, after, begin, count, jobs, offsets)) return false;
    std::size_t const hd = static_cast<std::size_t>(layout_.kv_head_count) * layout_.head_dimension;
    for (std::size_t k = first; k < jobs.size(); ++k) {
        kimkv_append_job& j = jobs[k];
        std::size_t const off = static_cast<std::size_t>(offsets[k - first]) * hd;
        j.src_key = input + off;
        j.src_value = input + static_cast<std::size_t>(count) * hd + off;
        j.src_layer_stride = 2ull * count * hd;
        j.src_token_stride = static_cast<std::uint32_t>(hd);
        j.layer_begin = 0;
        j.layer_count = layout_.layer_count;
    }
    return true;
}

HipStatus HipKvStorage::launchAppendJobs(std::vector<kimkv_append_job> const& jobs, HipStream stream)
{
    std::size_t const bytes = jobs.size() * sizeof(kimkv_append_job);
    HipStatus s{HipError::SubmissionFailed, 0};
    if (bytes <= ring_.capacity() / 2) {
        {
            std::lock_guard<std::mutex> lock(launch_mutex_);
            void* d = ring_.stage(jobs.data(), bytes, stream);
            if (d != nullptr) {
                s = mapStatus(kimkv_append_batch(storage_, static_cast<kimkv_append_job const*>(d),
                                                 static_cast<std::uint32_t>(jobs.size()), layout_.layer_count,
                                                 stream),
                              HipError::SubmissionFailed);
            } else {
                s = HipStatus{HipError::SubmissionFailed, kimkv_last_native_error()};
            }
            ring_.fence(stream);
        }
        return finish(stream, s);
    }
    TempDevice dev;   // larger than the staging ring: a one-off device copy
    if (!dev.upload(jobs.data(), bytes, stream)) {
        return finish(stream, HipStatus{HipError::SubmissionFailed, kimkv_last_native_error()});
    }
    s = mapStatus(kimkv_append_batch(storage_, static_cast<kimkv_append_job const*>(dev.mem.get()),
                                     static_cast<std::uint32_t>(jobs.size()), layout_.layer_count, stream),
                  HipError::SubmissionFailed);
    return finish(stream, s);
}

HipStatus HipKvStorage::append(BlockTable const& before, BlockTable const& after, std::uint32_t begin,
                               std::uint32_t count, KvScalar const* input, HipStream stream)
{
    if (!status_.ok()) return status_;
    if (consumeFailure(HipFailurePoint::Submission)) return HipStatus{HipError::SubmissionFailed, 0};
    std::vector<kimkv_append_job> jobs;
    if (!appendJobs(before, after, begin, count, input, jobs)) return HipStatus{HipError::InvalidArgument, 0};
    return launchAppendJobs(jobs, stream);
}

bool HipKvStorage::changeJobs(AppendChange const& change, std::uint32_t count, KvScalar const* input,
                              std::vector<kimkv_append_job>& jobs) const
{
    std::uint32_t const begin = change.logical_token_begin;
    std::uint64_t const end = static_cast<std::uint64_t>(begin) + count;
    if (input == nullptr || count == 0 || end > 0xFFFFFFFFull || change.entries.empty()
        || change.entries.front().logical_token_begin > begin) {
        return false;
    }
    bool const cow = change.replaced_tail.isStructurallyValid();
    if (cow) {
        // The private copy continues the replaced partial tail: its first
        // replaced_tokens tokens come from the source page, then the new ones.
        MappingEntry const& dst = change.entries.front();
        if (!pageExists(change.replaced_tail) || change.replaced_tail.kind != PageKind::Micro
            || dst.kind != PageKind::Micro || change.replaced_tokens == 0 || change.replaced_tokens >= micro_tokens_
            || static_cast<std::uint64_t>(dst.logical_token_begin) + change.replaced_tokens != begin) {
            return false;
        }
    }
    std::size_t const first = jobs.size();
    std::size_t const hd = static_cast<std::size_t>(layout_.kv_head_count) * layout_.head_dimension;
    std::uint64_t next = change.entries.front().logical_token_begin;
    for (std::size_t k = 0; k < change.entries.size(); ++k) {
        MappingEntry const& e = change.entries[k];
        kimkv_block_desc d{};
        if (!descriptor(e, d) || e.logical_token_begin != next) {
            jobs.resize(first);
            return false;
        }
        next += e.valid_tokens;
        std::uint32_t const sb = std::max(begin, e.logical_token_begin);
        std::uint32_t const se = static_cast<std::uint32_t>(std::min<std::uint64_t>(end, e.logicalTokenEnd()));
        if (sb >= se) continue;
        kimkv_append_job j{};
        std::size_t const off = static_cast<std::size_t>(sb - begin) * hd;
        j.src_key = input + off;
        j.src_value = input + static_cast<std::size_t>(count) * hd + off;
        j.src_layer_stride = 2ull * count * hd;
        j.src_token_stride = static_cast<std::uint32_t>(hd);
        j.layer_begin = 0;
        j.layer_count = layout_.layer_count;
        j.token_count = se - sb;
        j.dst_slot = e.handle.slot;
        j.dst_kind = static_cast<std::uint8_t>(e.kind);
        j.dst_token = static_cast<std::uint16_t>(sb - e.logical_token_begin);
        if (cow && k == 0) {
            j.cow_slot = change.replaced_tail.slot;
            j.cow_kind = static_cast<std::uint8_t>(change.replaced_tail.kind);
            j.cow_tokens = change.replaced_tokens;
        }
        jobs.push_back(j);
    }
    if (next != end || jobs.size() == first) {
        jobs.resize(first);
        return false;
    }
    return true;
}

HipStatus HipKvStorage::appendJobsNow(std::vector<kimkv_append_job> const& jobs, HipStream stream)
{
    if (!status_.ok()) return status_;
    if (consumeFailure(HipFailurePoint::Submission)) return HipStatus{HipError::SubmissionFailed, 0};
    if (jobs.empty()) return HipStatus{HipError::InvalidArgument, 0};
    return launchAppendJobs(jobs, stream);
}

HipStatus HipKvStorage::gather(BlockTable const& table, KvScalar* out, HipStream stream)
{
    if (!status_.ok()) return status_;
    if (consumeFailure(HipFailurePoint::Submission)) return HipStatus{HipError::SubmissionFailed, 0};
    if (out == nullptr || table.tokenCount() == 0 || !validTable(table)) return HipStatus{HipError::InvalidArgument, 0};
    std::vector<kimkv_block_desc> d;
    descriptors(table, d);
    TempDevice dev;
    if (!dev.upload(d.data(), d.size() * sizeof(kimkv_block_desc), stream)) {
        return finish(stream, HipStatus{HipError::SubmissionFailed, kimkv_last_native_error()});
    }
    HipStatus const s = mapStatus(kimkv_gather(storage_, static_cast<kimkv_block_desc const*>(dev.mem.get()),
                                               static_cast<std::uint32_t>(d.size()), table.tokenCount(), out, stream),
                                  HipError::SubmissionFailed);
    return finish(stream, s);
}

HipStatus HipKvStorage::promoteBatch(std::vector<PromotionPrepareResult> const& promotions, HipStream stream)
{
    if (!status_.ok()) return status_;
    if (consumeFailure(HipFailurePoint::Submission)) return HipStatus{HipError::SubmissionFailed, 0};
    if (micro_tokens_ != kMicroPageTokenCapacity || extent_tokens_ != kExtentPageTokenCapacity) {
        return HipStatus{HipError::InvalidArgument, 0};
    }
    std::vector<kimkv_promotion_job> jobs;
    for (PromotionPrepareResult const& p : promotions) {
        if (!p.ok() || p.target_handle.kind != PageKind::Extent || !pageExists(p.target_handle)) {
            return HipStatus{HipError::InvalidArgument, 0};
        }
        kimkv_promotion_job j{};
        for (std::size_t i = 0; i < kPromotionSourcePageCount; ++i) {
            PageHandle const s = p.source_handles[i];
            if (s.kind != PageKind::Micro || !pageExists(s)) return HipStatus{HipError::InvalidArgument, 0};
            j.micro_slots[i] = s.slot;
        }
        j.extent_slot = p.target_handle.slot;
        jobs.push_back(j);
    }
    if (jobs.empty()) return {};
    TempDevice dev;
    if (!dev.upload(jobs.data(), jobs.size() * sizeof(kimkv_promotion_job), stream)) {
        return finish(stream, HipStatus{HipError::SubmissionFailed, kimkv_last_native_error()});
    }
    HipStatus const s = mapStatus(kimkv_promote_batch(storage_, static_cast<kimkv_promotion_job const*>(dev.mem.get()),
                                                      static_cast<std::uint32_t>(jobs.size()), stream),
                                  HipError::SubmissionFailed);
    return finish(stream, s);
}

HipStatus HipKvStorage::promote(PromotionPrepareResult const& promotion, HipStream stream)
{
    return promoteBatch(std::vector<PromotionPrepareResult>{promotion}, stream);
}

HipStatus HipKvStorage::referenceAttention(BlockTable const& table, float const* query, float* output,
                                           HipStream stream)
{
    if (!status_.ok()) return status_;
    if (consumeFailure(HipFailurePoint::Submission)) return HipStatus{HipError::SubmissionFailed, 0};
    if (query == nullptr || output == nullptr || table.tokenCount() == 0 || !validTable(table)) {
        return HipStatus{HipError::InvalidArgument, 0};
    }
    std::vector<kimkv_block_desc> d;
    descriptors(table, d);
    TempDevice dev;
    if (!dev.upload(d.data(), d.size() * sizeof(kimkv_block_desc), stream)) {
        return finish(stream, HipStatus{HipError::SubmissionFailed, kimkv_last_native_error()});
    }
    HipStatus const s = mapStatus(
        kimkv_reference_attention(storage_, static_cast<kimkv_block_desc const*>(dev.mem.get()),
                                  static_cast<std::uint32_t>(d.size()), table.tokenCount(), query, output, stream),
        HipError::SubmissionFailed);
    return finish(stream, s);
}

}  // namespace kimkvcache
