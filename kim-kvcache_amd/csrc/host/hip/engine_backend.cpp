// Heterogeneous engine backend on MI355X.
//
// Behaviour follows the reference's CUDA backend (src/cuda/engine/backend.cpp:
// 19-610 and transaction.cpp:24-423): reserve = metadata reservation +
// device descriptors; writeLayer / attendLayer only enqueue; commit waits on
// one completion event and publishes the table; any failure rolls back after
// in-flight work has drained; error codes map as in backend.cpp:19-65.
// Differences: a reservation costs O(1) in the context length -- the manager
// reserves by tail delta, each request's table stays resident on the device
// and only its tail entry is patched (the reference copies both tables,
// leases every page and uploads the whole table per token); batched
// attention has no lane cap and one decode launch covers every lane;
// writeLayerBatch appends all lanes in one launch; small per-launch uploads go
// through a pinned staging ring instead of cudaMalloc per token.
#include "kim-kv/hip/hip_engine_kv_backend.h"

#include "kim-kv/runtime/kv_cache_manager.h"
#include "kim-kv/runtime/pool_permutation.h"
#include "storage.h"

#include <algorithm>
#include <deque>
#include <atomic>
#include <cstddef>
#include <cstring>
#include <optional>
#include <memory>
#include <mutex>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace kimkvcache {
namespace {

EngineKvStatus mapMetadata(KvCacheError e) noexcept
{
    switch (e) {
    case KvCacheError::None: return {};
    case KvCacheError::InvalidArgument: return {EngineKvError::InvalidArgument};
    case KvCacheError::RequestNotFound: return {EngineKvError::RequestNotFound};
    case KvCacheError::RequestAlreadyExists: return {EngineKvError::RequestAlreadyExists};
    case KvCacheError::RequestConflict:
    case KvCacheError::PromotionConflict: return {EngineKvError::RequestConflict};
    case KvCacheError::ResourceExhausted: return {EngineKvError::ResourceExhausted};
    case KvCacheError::InvalidState: return {EngineKvError::InvalidState};
    default: return {EngineKvError::InternalError};
    }
}

EngineKvStatus mapDevice(HipStatus s) noexcept
{
    switch (s.error) {
    case HipError::None: return {};
    case HipError::InvalidArgument: return {EngineKvError::InvalidArgument};
    case HipError::AllocationFailed: return {EngineKvError::ResourceExhausted};
    case HipError::SubmissionFailed: return {EngineKvError::SubmissionFailed};
    case HipError::ExecutionFailed: return {EngineKvError::ExecutionFailed};
    default: return {EngineKvError::InternalError};
    }
}

HipStatus invalidArgument() noexcept { return HipStatus{HipError::InvalidArgument, 0}; }
HipStatus injectedSubmission() noexcept { return HipStatus{HipError::SubmissionFailed, 0}; }

constexpr std::uint64_t kStaleTable = ~std::uint64_t{0};

// A request's committed block table kept in device memory across tokens: a
// token reservation patches its tail entry instead of uploading the table.
// `version` is the manager table version the copy holds, kStaleTable while a
// reservation's candidate is patched in or after a failure; a reservation
// that finds it stale (or too small) rewrites it whole.  Only the request's
// own token transactions read it, and each of them waits for its device work
// before it resolves, which the manager requires before the request's next
// reservation, append, promotion or release: the copy is rewritten or freed
// without a fence.
struct DeviceTable final {
    DeviceBufferCache* cache{nullptr};
    kimkv_block_desc* ptr{nullptr};
    std::size_t granted{0};
    std::uint64_t version{kStaleTable};

    DeviceTable() = default;
    DeviceTable(DeviceTable const&) = delete;
    DeviceTable& operator=(DeviceTable const&) = delete;
    DeviceTable(DeviceTable&& o) noexcept : cache(o.cache), ptr(o.ptr), granted(o.granted), version(o.version)
    {
        o.ptr = nullptr;
        o.granted = 0;
    }
    DeviceTable& operator=(DeviceTable&&) = delete;
    ~DeviceTable() { reset(); }

    [[nodiscard]] std::uint32_t capacity() const noexcept
    {
        return static_cast<std::uint32_t>(std::min<std::size_t>(granted / sizeof(kimkv_block_desc), 0xFFFFFFFFu));
    }
    void reset() noexcept
    {
        if (ptr != nullptr) cache->release(ptr, granted);
        ptr = nullptr;
        granted = 0;
        version = kStaleTable;
    }
    // Room for `entries` (plus headroom for the next tokens); false when out
    // of device memory (the copy is then released and stale).
    bool fit(DeviceBufferCache& buffers, std::uint32_t entries) noexcept
    {
        if (ptr != nullptr && capacity() >= entries) return true;
        reset();
        std::size_t const want = (static_cast<std::size_t>(entries) + std::max<std::size_t>(entries / 4, 32))
            * sizeof(kimkv_block_desc);
        void* mem = nullptr;
        try {
            mem = buffers.acquire(want, granted);
        } catch (...) {
            mem = nullptr;
        }
        if (mem == nullptr) {
            granted = 0;
            return false;
        }
        cache = &buffers;
        ptr = static_cast<kimkv_block_desc*>(mem);
        return true;
    }
};

struct RequestState final {
    std::uint32_t length{0};   // committed tokens
    DeviceTable table;
};

// One lane of a batched attention launch from device lane records
// (kimkv_paged_decode_lanes), without its chunk range: its request's table,
// its token count and the single-token write the launch stores (none when
// w.token_count is 0).
kimkv_decode_lane laneRecordOf(kimkv_block_desc const* table, std::uint32_t count, std::uint32_t tokens,
                               kimkv_append_job const& w) noexcept
{
    kimkv_decode_lane r{};
    r.descriptors = table;
    r.descriptor_count = count;
    r.token_count = tokens;
    if (w.token_count != 0) {
        r.dst_slot = w.dst_slot;
        r.cow_slot = w.cow_slot;
        r.dst_token = w.dst_token;
        r.cow_tokens = w.cow_tokens;
        r.dst_kind = w.dst_kind;
        r.cow_kind = w.cow_kind;
        r.has_write = 1;
    }
    return r;
}

// The key of a launch's chunk records: each lane's record with its chunk
// range from the plan's prefix, then the planned chunk flags (so that a copy
// stands for one plan).
void laneRecordKey(std::vector<kimkv_decode_lane> const& lanes, std::vector<std::uint32_t> const& pre,
                   std::uint32_t chunk, std::vector<unsigned char>& out)
{
    std::size_t const n = lanes.size();
    out.assign(n * sizeof(kimkv_decode_lane) + sizeof(std::uint32_t), 0);
    for (std::size_t i = 0; i < n; ++i) {
        kimkv_decode_lane r = lanes[i];
        r.lane = static_cast<std::uint32_t>(i);
        r.first_chunk = pre[i];
        r.chunk_count = pre[i + 1] - pre[i];
        std::memcpy(out.data() + i * sizeof(r), &r, sizeof(r));
    }
    std::memcpy(out.data() + n * sizeof(kimkv_decode_lane), &chunk, sizeof(chunk));
}

// The chunk records of a key: each lane's record repeated over its chunks
// (total_chunks records), padded with zeros to a whole number of
// descriptors (the unit the reserve call's patch launch copies).  False when
// a lane's range lies outside the launch.
bool expandLaneRecords(std::vector<unsigned char> const& key, std::uint32_t total_chunks,
                       std::vector<kimkv_block_desc>& out)
{
    std::size_t const rec = sizeof(kimkv_decode_lane);
    std::size_t const lanes = (key.size() - sizeof(std::uint32_t)) / rec;
    std::size_t const bytes = static_cast<std::size_t>(total_chunks) * rec;
    out.assign((bytes + sizeof(kimkv_block_desc) - 1) / sizeof(kimkv_block_desc), kimkv_block_desc{});
    auto* dst = reinterpret_cast<unsigned char*>(out.data());
    for (std::size_t i = 0; i < lanes; ++i) {
        kimkv_decode_lane r;
        std::memcpy(&r, key.data() + i * rec, rec);
        if (static_cast<std::uint64_t>(r.first_chunk) + r.chunk_count > total_chunks) return false;
        for (std::uint32_t k = 0; k < r.chunk_count; ++k) {
            std::memcpy(dst + (static_cast<std::size_t>(r.first_chunk) + k) * rec, &r, rec);
        }
    }
    return true;
}

struct BackendState final {
    EngineKvConfig config;
    KvCacheManager manager;
    HipKvStorage storage;
    std::unordered_map<RequestId, RequestState> requests;
    // Requests with an unfinished PrefillChunk: their table already holds the
    // chunk, so every other mutation of them is refused until finish().
    std::unordered_set<RequestId> prefilling;
    std::uint64_t active_transactions{0};
    std::atomic<std::uint64_t> batched_attention_submissions{0};
    std::atomic<std::uint64_t> batched_attention_lanes{0};
    std::atomic<std::uint64_t> batched_write_submissions{0};
    std::atomic<std::uint64_t> lane_record_launches{0};   // of batched_attention_submissions
    std::atomic<std::uint64_t> next_transaction_id{1};
    mutable std::mutex mutex;
    std::mutex event_mutex;
    std::vector<void*> free_events;   // completion events of finished transactions

    // Device copies of the chunk records (kimkv_decode_lane, one per chunk)
    // of recent batched attention launches, a few per stream, each keyed by
    // its lanes' records and plan (one record per lane, then the chunk
    // flags).  The layers of a token step launch the same lanes with the same
    // records: a reserve call copies the records of its transactions in
    // reservation order with its descriptor patches; an attention that
    // misses them copies its own at layer 0 of a model with more layers, or
    // else when a stream asks for the same key a second time (a one-layer
    // step never pays for a separate copy); later layers reuse the copy.  An
    // entry is written only by
    // copies on its own stream, which run after that stream's earlier
    // launches that read it; a buffer is replaced only after its stream has
    // drained.  Guarded by the storage's launch mutex.
    struct LaneRecords {
        HipStream stream{nullptr};
        std::vector<unsigned char> key;   // what `device` was expanded from
        DeviceMemory device;
        std::uint64_t device_bytes{0};
        std::uint64_t used{0};
        // The chunk group tables of launches from these records
        // (kimkv_paged_decode_lanes' table cache), tagged per copy of them
        // and again after any block-table write on the storage.
        std::uint32_t tag{0};
        std::uint64_t tag_writes{0};   // the storage's descriptorWrites() when tagged
        DeviceMemory tables;
        std::uint64_t tables_bytes{0};
    };
    static constexpr std::uint32_t kTableCacheMaxChunk = 4096;   // tokens
    std::uint32_t last_table_tag{0};
    struct LaneRecordsSeen {
        HipStream stream{nullptr};
        std::vector<unsigned char> key;   // the stream's last request without a copy
    };
    std::vector<LaneRecordsSeen> lane_records_seen;
    static constexpr std::size_t kLaneRecordsPerStream = 4;
    static constexpr std::size_t kLaneRecordEntries = 64;
    std::deque<LaneRecords> lane_records;   // grows only; entries keep their addresses
    std::uint64_t lane_record_clock{0};

    // Grows `mem` (capacity `bytes`) to at least `need` bytes for work on
    // `stream`, draining the stream first when a buffer is replaced.  Sizes
    // leave headroom (at least 64 KiB, 1.5x the need, twice the old size):
    // a batch's chunk count creeps up as its lanes grow, and each
    // replacement waits for the stream.
    static bool growDevice(DeviceMemory& mem, std::uint64_t& bytes, std::uint64_t need, HipStream stream)
    {
        if (bytes >= need) return true;
        if (mem.get() != nullptr && kimkv_stream_synchronize(stream) != KIMKV_OK) return false;
        std::uint64_t const grown = std::max<std::uint64_t>({need + need / 2, 2 * bytes, std::uint64_t{64} << 10});
        mem = DeviceMemory(grown);
        bytes = mem.get() != nullptr ? grown : 0;
        return mem.get() != nullptr;
    }

    // The least recently used entry of `stream`, or a new one while the
    // stream has fewer than kLaneRecordsPerStream; nullptr when none can be
    // had.  Its contents are unknown from here on (key cleared).
    LaneRecords* laneRecordsVictim(HipStream stream)
    {
        LaneRecords* victim = nullptr;
        std::size_t mine = 0;
        for (LaneRecords& e : lane_records) {
            if (e.stream != stream) continue;
            ++mine;
            if (victim == nullptr || e.used < victim->used) victim = &e;
        }
        if (mine < kLaneRecordsPerStream && lane_records.size() < kLaneRecordEntries) {
            LaneRecords e;
            e.stream = stream;
            lane_records.push_back(std::move(e));
            victim = &lane_records.back();
        }
        if (victim != nullptr) victim->key.clear();
        return victim;
    }

    // The entry holding the chunk records of `key` (lane records, then the
    // chunk flags) for launches on `stream`: one already holding them (a
    // reserve call may have copied them), or, when the stream asked for the
    // same key last time or the caller expects it again (`reused`: later
    // layers of the step follow), one of the stream's entries refilled by a
    // copy on the stream.  nullptr otherwise (the caller stages the launch
    // another way).
    LaneRecords* laneRecords(std::vector<unsigned char> const& key, std::uint32_t total_chunks, HipStream stream,
                             bool reused)
    {
        for (LaneRecords& e : lane_records) {
            if (e.stream == stream && e.key == key) {
                e.used = ++lane_record_clock;
                retag(e, false);
                return &e;
            }
        }
        LaneRecordsSeen* seen = nullptr;
        for (LaneRecordsSeen& e : lane_records_seen) {
            if (e.stream == stream) seen = &e;
        }
        if (seen == nullptr) {
            if (lane_records_seen.size() >= kLaneRecordEntries) return nullptr;
            lane_records_seen.push_back(LaneRecordsSeen{stream, {}});
            seen = &lane_records_seen.back();
        }
        if (seen->key != key && !reused) {   // first request: remember it, copy nothing yet
            seen->key = key;
            return nullptr;
        }
        seen->key.clear();
        thread_local std::vector<kimkv_block_desc> chunks;
        if (!expandLaneRecords(key, total_chunks, chunks)) return nullptr;
        std::size_t const bytes = chunks.size() * sizeof(kimkv_block_desc);
        LaneRecords* victim = laneRecordsVictim(stream);
        if (victim == nullptr || !growDevice(victim->device, victim->device_bytes, bytes, stream)
            || !storage.ring().uploadTo(victim->device.get(), chunks.data(), bytes, stream)) {
            return nullptr;
        }
        victim->key = key;
        victim->used = ++lane_record_clock;
        retag(*victim, true);
        return victim;
    }

    // An entry of `stream` for the chunk records of `key` that the caller
    // copies into it before anything else runs on the stream (a reserve
    // call's patch launch): grown to `bytes`, keyed and freshly tagged.
    // nullptr when no entry or memory can be had.  Under the launch mutex.
    LaneRecords* seedLaneRecords(std::vector<unsigned char> const& key, std::uint64_t bytes, HipStream stream)
    {
        for (LaneRecords& e : lane_records) {
            if (e.stream == stream && e.key == key) e.key.clear();   // one entry per key
        }
        LaneRecords* victim = laneRecordsVictim(stream);
        if (victim == nullptr || !growDevice(victim->device, victim->device_bytes, bytes, stream)) return nullptr;
        victim->key = key;
        victim->used = ++lane_record_clock;
        retag(*victim, true);
        return victim;
    }

    // A fresh table tag (never 0) for new records, or when a block table may
    // have changed since the entry was tagged: a tag names one set of
    // records over unchanged tables.  Under the storage's launch mutex.
    void retag(LaneRecords& e, bool fresh_records)
    {
        std::uint64_t const writes = storage.descriptorWrites();
        if (!fresh_records && e.tag != 0 && e.tag_writes == writes) return;
        e.tag = ++last_table_tag == 0 ? ++last_table_tag : last_table_tag;
        e.tag_writes = writes;
    }

    // The entry's table cache for a launch of total_chunks chunks planned
    // with chunk_flags (grown, and zeroed, on the entry's stream when too
    // small), or nullptr when chunks are too long to cache or memory is short.
    void* laneTables(LaneRecords& e, std::uint32_t total_chunks, std::uint32_t chunk_flags, std::uint64_t& bytes)
    {
        std::uint32_t const chunk = chunk_flags & ~(KIMKV_DECODE_HEAD_SPLIT | KIMKV_DECODE_GUIDED);
        if (chunk > kTableCacheMaxChunk) return nullptr;
        std::uint64_t const need = kimkv_decode_table_cache_bytes(total_chunks, chunk_flags);
        if (e.tables_bytes < need) {
            // A new buffer starts zeroed: tag 0 is never a launch's.
            if (!growDevice(e.tables, e.tables_bytes, need, e.stream)
                || kimkv_fill_f16(static_cast<std::uint16_t*>(e.tables.get()), e.tables_bytes / 2, 0, e.stream)
                       != KIMKV_OK) {
                e.tables_bytes = 0;
                return nullptr;
            }
        }
        bytes = e.tables_bytes;
        return e.tables.get();
    }

    BackendState(EngineKvConfig c, std::uint32_t micro, std::uint32_t extent)
        : config(c), manager(micro, extent), storage(c.kv_layout, micro, extent)
    {
    }

    ~BackendState()
    {
        for (void* e : free_events) static_cast<void>(kimkv_event_destroy(e));
    }

    // Completion events are recycled: creating one per token costs more than
    // the rest of a reserve.
    void* acquireEvent() noexcept
    {
        {
            std::lock_guard<std::mutex> lock(event_mutex);
            if (!free_events.empty()) {
                void* e = free_events.back();
                free_events.pop_back();
                return e;
            }
        }
        void* e = nullptr;
        return kimkv_event_create(&e, 0) == KIMKV_OK ? e : nullptr;
    }

    // Only events that have been waited for (or never recorded) come back.
    void releaseEvent(void* e) noexcept
    {
        if (e == nullptr) return;
        std::lock_guard<std::mutex> lock(event_mutex);
        try {
            free_events.push_back(e);
        } catch (...) {
            static_cast<void>(kimkv_event_destroy(e));
        }
    }
};

// Completion of one launch, shared by every transaction in it: an event
// recorded right after the launch.  Commit waits on the mark of the
// transaction's last launch rather than on an event recorded at commit time,
// so committing one lane group is not held up by work queued after it on the
// same stream (the next group's layers).
struct CompletionMark final {
    std::shared_ptr<BackendState> owner;
    void* event{nullptr};

    CompletionMark(std::shared_ptr<BackendState> o, void* e) : owner(std::move(o)), event(e) {}
    ~CompletionMark() { owner->releaseEvent(event); }
    CompletionMark(CompletionMark const&) = delete;
    CompletionMark& operator=(CompletionMark const&) = delete;
};

std::shared_ptr<CompletionMark> markLaunch(std::shared_ptr<BackendState> const& owner, HipStream stream) noexcept
{
    void* e = owner->acquireEvent();
    if (e == nullptr) return nullptr;
    if (kimkv_event_record(e, stream) != KIMKV_OK) {
        owner->releaseEvent(e);
        return nullptr;
    }
    try {
        return std::make_shared<CompletionMark>(owner, e);
    } catch (...) {
        owner->releaseEvent(e);
        return nullptr;
    }
}

// Device block descriptors of one reserve call: every transaction of a
// batched reserve points into one arena filled by a single upload; the
// buffer returns to the cache when the last of them has finished.
struct DescriptorArena final {
    std::shared_ptr<BackendState> owner;
    void* ptr{nullptr};
    std::size_t granted{0};

    DescriptorArena(std::shared_ptr<BackendState> o, void* p, std::size_t g) : owner(std::move(o)), ptr(p), granted(g) {}
    ~DescriptorArena() { owner->storage.buffers().release(ptr, granted); }
    DescriptorArena(DescriptorArena const&) = delete;
    DescriptorArena& operator=(DescriptorArena const&) = delete;
};

class HipTokenTransaction final : public TokenTransactionBackend {
public:
    HipTokenTransaction(std::shared_ptr<BackendState> owner, TokenReservationDelta const& r, HipStream stream)
        : owner_(std::move(owner)),
          reservation_(r.reservation_id),
          request_(r.request_id),
          committed_version_(r.committed_version),
          stream_(stream),
          token_count_(r.logical_token_position + 1)
    {
        tail_ = r.tail.handle;
        tail_token_ = static_cast<std::uint16_t>(token_count_ - 1 - r.tail.logical_token_begin);
        if (!r.appended && r.has_previous_tail && r.previous_tail.handle != r.tail.handle) {
            cow_src_ = r.previous_tail.handle;   // partial tail replaced: copy per layer
            cow_tokens_ = r.previous_tail.valid_tokens;
        }
    }

    ~HipTokenTransaction() override
    {
        static_cast<void>(finish());
        releaseDescriptors();
    }

    // Binds the transaction to its request's device table, whose candidate
    // patch the reserve call has enqueued on this transaction's stream.
    void attach(kimkv_block_desc const* table, std::uint32_t count) noexcept
    {
        table_ = table;
        descriptors_ = table;
        desc_count_ = count;
        dirty_ = true;   // the patch is in flight
        submission_ = {};
    }

    EngineKvStatus writeLayer(LayerKvWrite const& write, EngineStream) override
    {
        kimkv_append_job job{};
        HipStatus s = prepareWrite(write, job);
        if (!s.ok()) return mapDevice(s);
        holdWrite(job);
        return {};
    }

    EngineKvStatus attendLayer(PagedDecodeRequest const& request, EngineStream) override
    {
        kimkv_decode_item item{};
        std::vector<std::uint32_t> prefix(2, 0);
        std::uint32_t chunk = 0;
        std::uint32_t total = 0;
        HipStatus s = planOne(request, item, prefix, chunk, total);
        if (!s.ok()) return mapDevice(s);
        std::lock_guard<std::mutex> lock(owner_->storage.launchMutex());
        HipKvStorage& st = owner_->storage;
        struct {
            kimkv_decode_item item;
            kimkv_append_job write;
            std::uint32_t prefix[2];
        } packed{item, takeWrite(), {prefix[0], prefix[1]}};
        auto* staged = static_cast<unsigned char*>(st.ring().stage(&packed, sizeof(packed), stream_));
        if (staged == nullptr) return mapDevice(failSubmission(kimkv_last_native_error()));
        kimkv_status const k = kimkv_paged_decode_write_batch(
            st.handle(), reinterpret_cast<kimkv_decode_item const*>(staged),
            reinterpret_cast<std::uint32_t const*>(staged + offsetof(decltype(packed), prefix)), 1, total, chunk,
            owner_->config.query_head_count,
            reinterpret_cast<kimkv_append_job const*>(staged + offsetof(decltype(packed), write)), stream_);
        st.ring().fence(stream_);
        if (k != KIMKV_OK) return mapDevice(failSubmission(kimkv_last_native_error()));
        dirty_ = true;
        if (request.layer + 1 == owner_->config.kv_layout.layer_count) setMark(markLaunch(owner_, stream_));
        return {};
    }

    // The per-layer arguments of kimkv_paged_decode_lanes for the first n
    // launched lanes: true when they attend one layer with one scale, every
    // lane or none writes a token (a one-token, one-layer job), and each of
    // their queries, outputs, workspaces and new K / V rows sits at base +
    // lane * stride.  Lanes whose chunk needs no workspace get the evenly
    // spaced address too; the kernel uses it only for multi-chunk lanes,
    // whose workspaces were checked.
    static bool evenLayerArgs(PagedDecodeBatch const& batch, std::vector<std::size_t> const& launched,
                              std::vector<kimkv_append_job> const& writes, std::size_t n,
                              kimkv_decode_layer_args& a)
    {
        DevicePagedDecodeBatchItem const* h = batch.host_items;
        bool const writing = writes[0].token_count != 0;
        for (std::size_t i = 0; i < n; ++i) {
            kimkv_append_job const& w = writes[i];
            if (h[i].layer != h[0].layer || h[i].attention_scale != h[0].attention_scale
                || (w.token_count != 0) != writing) {
                return false;
            }
            if (writing && (w.token_count != 1 || w.layer_count != 1 || w.layer_begin != h[i].layer
                            || w.src_layer_stride != 0 || w.src_token_stride != 0)) {
                return false;
            }
        }
        auto even = [n](auto at, auto& base, std::uint64_t& stride) {
            auto const b = reinterpret_cast<std::uintptr_t>(at(0));
            stride = n > 1 ? static_cast<std::uint64_t>(reinterpret_cast<std::uintptr_t>(at(1)) - b) : 0;
            for (std::size_t i = 2; i < n; ++i) {
                if (reinterpret_cast<std::uintptr_t>(at(i)) != b + stride * i) return false;
            }
            base = at(0);
            return true;
        };
        a = kimkv_decode_layer_args{};
        a.layer = h[0].layer;
        a.attention_scale = h[0].attention_scale;
        bool ok = even([h](std::size_t i) { return reinterpret_cast<std::uint16_t const*>(h[i].device_query); },
                       a.query, a.query_stride)
            && even([h](std::size_t i) { return reinterpret_cast<std::uint16_t*>(h[i].device_output); }, a.output,
                    a.output_stride)
            && even([&](std::size_t i) { return static_cast<float*>(batch.items[launched[i]].request.device_workspace); },
                    a.workspace, a.workspace_stride);
        if (ok && writing) {
            ok = even([&](std::size_t i) { return writes[i].src_key; }, a.key, a.key_stride)
                && even([&](std::size_t i) { return writes[i].src_value; }, a.value, a.value_stride);
        }
        return ok;
    }

    // The key of the first n launched lanes' chunk records (laneRecordKey).
    static void laneRecordBytes(DevicePagedDecodeBatchItem const* h, std::vector<kimkv_append_job> const& writes,
                                std::vector<std::uint32_t> const& pre, std::uint32_t chunk, std::size_t n,
                                std::vector<unsigned char>& out)
    {
        thread_local std::vector<kimkv_decode_lane> lanes;
        lanes.resize(n);
        for (std::size_t i = 0; i < n; ++i) {
            lanes[i] = laneRecordOf(reinterpret_cast<kimkv_block_desc const*>(h[i].device_descriptors),
                                    h[i].descriptor_count, h[i].token_count, writes[i]);
        }
        laneRecordKey(lanes, pre, chunk, out);
    }

    // This transaction's lane record as its attention launches from device
    // lane records will read it, once attached to `table` (`count` entries):
    // every layer's attention stores the layer's token (writeLayer must
    // precede it), at the destination the reservation fixed.
    kimkv_decode_lane plannedLaneRecord(kimkv_block_desc const* table, std::uint32_t count) const noexcept
    {
        kimkv_append_job job{};
        job.token_count = 1;
        job.dst_slot = tail_.slot;
        job.dst_kind = static_cast<std::uint8_t>(tail_.kind);
        job.dst_token = tail_token_;
        if (cow_tokens_ != 0) {
            job.cow_slot = cow_src_.slot;
            job.cow_kind = static_cast<std::uint8_t>(cow_src_.kind);
            job.cow_tokens = cow_tokens_;
        }
        return laneRecordOf(table, count, token_count_, job);
    }

    std::uint32_t tokenCount() const noexcept { return token_count_; }

    void attendLayerBatch(PagedDecodeBatch& batch) override
    {
        std::vector<HipTokenTransaction*> lanes;
        std::vector<std::size_t> index;
        if (!collect(batch, lanes, index)) {
            TokenTransactionBackend::attendLayerBatch(batch);
            return;
        }
        BackendState& o = *owner_;
        HipKvStorage& st = o.storage;
        std::uint32_t const QH = o.config.query_head_count;
        std::uint32_t const D = o.config.kv_layout.head_dimension;
        // Prepare every lane (per-lane validation, fault hook) before planning.
        std::vector<std::uint32_t> tokens;
        std::vector<std::size_t> ready;
        for (std::size_t k = 0; k < lanes.size(); ++k) {
            PagedDecodeBatchItem& item = batch.items[index[k]];
            HipStatus const s = lanes[k]->checkAttention(item.request);
            if (!s.ok()) {
                item.status = mapDevice(s);
                continue;
            }
            ready.push_back(k);
            tokens.push_back(lanes[k]->token_count_);
        }
        if (ready.empty()) return;
        std::vector<std::uint32_t> prefix(ready.size() + 1, 0);
        std::uint32_t chunk = 0;
        std::uint32_t total = 0;
        if (kimkv_decode_plan(st.handle(), tokens.data(), static_cast<std::uint32_t>(ready.size()), QH, &chunk,
                              prefix.data(), &total) != KIMKV_OK) {
            for (std::size_t k : ready) batch.items[index[k]].status = {EngineKvError::InvalidArgument};
            return;
        }
        std::size_t n = 0;
        std::vector<std::size_t> launched;
        std::vector<std::uint32_t> launch_prefix(1, 0);
        std::vector<std::uint32_t> launch_tokens;
        thread_local std::vector<kimkv_append_job> writes;
        writes.clear();
        for (std::size_t k : ready) {
            PagedDecodeBatchItem& item = batch.items[index[k]];
            HipTokenTransaction* t = lanes[k];
            std::size_t const need = kimkv_decode_workspace_bytes(t->token_count_, chunk, QH, D);
            if (item.request.workspace_bytes < need) {
                item.status = {EngineKvError::InvalidArgument};
                continue;
            }
            batch.host_items[n] = t->deviceItem(item.request, need != 0);
            writes.push_back(t->takeWrite());   // this layer's token, written by the launch
            launched.push_back(index[k]);
            launch_tokens.push_back(t->token_count_);
            ++n;
        }
        if (n == 0) return;
        // Prefix over the surviving lanes with the chunk length their workspaces
        // were checked against (re-planning could shrink it and overflow them).
        std::vector<std::uint32_t> pre(n + 1, 0);
        for (std::size_t i = 0; i < n; ++i) pre[i + 1] = pre[i] + kimkv_decode_lane_chunks(launch_tokens[i], chunk, D);
        total = pre[n];
        std::lock_guard<std::mutex> lock(o.storage.launchMutex());
        HipStream const stream = stream_;
        kimkv_status k = KIMKV_SUBMISSION_FAILED;
        bool launched_from_records = false;
        kimkv_decode_layer_args args{};
        if (n <= KIMKV_DECODE_ARG_PREFIX_LANES && evenLayerArgs(batch, launched, writes, n, args)
            && (total == n || args.workspace != nullptr)) {
            // Every chunk's step-constant record from a device copy (made by
            // the reserve call, or here): no workgroup reads host memory
            // before its block table.
            thread_local std::vector<unsigned char> records;
            laneRecordBytes(batch.host_items, writes, pre, chunk, n, records);
            // Layer 0 of a model with more layers copies the records at once
            // (the step's other layers reuse them); otherwise only a batch
            // the stream asks for twice is copied, so a one-layer step
            // never pays for a copy.
            bool const first_of_many = args.layer == 0 && o.config.kv_layout.layer_count > 1;
            BackendState::LaneRecords* rec = o.laneRecords(records, total, stream, first_of_many);
            if (rec != nullptr) {
                // Chunk group tables cached per copy of the records: built
                // by the first launch from them, read by the later layers.
                // The merge takes the lanes' chunk counts from the prefix in
                // its arguments (no merge records).
                std::uint64_t table_bytes = 0;
                void* tables = o.laneTables(*rec, total, chunk, table_bytes);
                k = kimkv_paged_decode_lanes(st.handle(), static_cast<kimkv_decode_lane const*>(rec->device.get()),
                                             static_cast<std::uint32_t>(n), total, chunk, QH, &args, pre.data(),
                                             nullptr, tables, table_bytes, tables != nullptr ? rec->tag : 0, stream);
                launched_from_records = true;
                if (k == KIMKV_OK) o.lane_record_launches.fetch_add(1, std::memory_order_relaxed);
            }
        }
        // Otherwise items, write jobs and chunk prefix are staged together in
        // pinned host memory that the kernels read directly (a copy command
        // on the stream would cost a dispatch and a gap between kernels); the
        // caller's device_items scratch is validated by the API but not
        // needed here.
        std::size_t const items_bytes = (n * sizeof(DevicePagedDecodeBatchItem) + 15) & ~std::size_t{15};
        std::size_t const writes_bytes = n * sizeof(kimkv_append_job);
        std::size_t const prefix_at = items_bytes + ((writes_bytes + 15) & ~std::size_t{15});
        thread_local std::vector<unsigned char> staging;
        unsigned char* staged = nullptr;
        if (!launched_from_records) {
            staging.resize(prefix_at + pre.size() * 4);
            std::memcpy(staging.data(), batch.host_items, n * sizeof(DevicePagedDecodeBatchItem));
            std::memcpy(staging.data() + items_bytes, writes.data(), writes_bytes);
            std::memcpy(staging.data() + prefix_at, pre.data(), pre.size() * 4);
            staged = static_cast<unsigned char*>(st.ring().stage(staging.data(), staging.size(), stream));
        }
        if (staged != nullptr) {
            // With split-K lanes, the merge launch reads its per-lane records
            // from device scratch the decode launch fills, not the staged
            // items (a round trip to host memory at its start).
            void* slots = total > n ? st.ring().deviceScratch(n * KIMKV_DECODE_LANE_SLOT_BYTES, stream) : nullptr;
            auto const* items_d = reinterpret_cast<kimkv_decode_item const*>(staged);
            auto const* prefix_d = reinterpret_cast<std::uint32_t const*>(staged + prefix_at);
            auto const* writes_d = reinterpret_cast<kimkv_append_job const*>(staged + items_bytes);
            // Small batches also carry the chunk prefix in the launch's
            // arguments: every workgroup finds its lane without a round trip
            // to the staged prefix (ragged lanes miss the kernel's guess).
            k = slots != nullptr
                ? kimkv_paged_decode_write_batch_slots_prefix(st.handle(), items_d, prefix_d, pre.data(),
                                                              static_cast<std::uint32_t>(n), total, chunk, QH,
                                                              writes_d, slots, stream)
                : kimkv_paged_decode_write_batch(st.handle(), items_d, prefix_d, static_cast<std::uint32_t>(n),
                                                 total, chunk, QH, writes_d, stream);
        }
        st.ring().fence(stream);
        // Only the last layer's launch needs a completion mark (commit waits
        // on it); earlier launches leave the transactions dirty.
        bool last_layer = false;
        for (std::size_t i : launched) {
            last_layer = last_layer || batch.items[i].request.layer + 1 == o.config.kv_layout.layer_count;
        }
        std::shared_ptr<CompletionMark> const mark = k == KIMKV_OK && last_layer ? markLaunch(owner_, stream) : nullptr;
        std::uint64_t good = 0;
        for (std::size_t i : launched) {
            PagedDecodeBatchItem& item = batch.items[i];
            auto* t = static_cast<HipTokenTransaction*>(batchBackend(item));
            item.status = k == KIMKV_OK ? EngineKvStatus{} : mapDevice(t->failSubmission(kimkv_last_native_error()));
            if (k == KIMKV_OK) {
                t->dirty_ = true;
                if (item.request.layer + 1 == o.config.kv_layout.layer_count) t->setMark(mark);
            }
            good += item.status.ok() ? 1 : 0;
        }
        if (good != 0) {
            o.batched_attention_submissions.fetch_add(1, std::memory_order_relaxed);
            o.batched_attention_lanes.fetch_add(good, std::memory_order_relaxed);
        }
    }

    void writeLayerBatch(LayerKvWriteBatch& batch) override
    {
        std::vector<HipTokenTransaction*> lanes;
        std::vector<std::size_t> index;
        for (std::size_t i = 0; i < batch.item_count; ++i) {
            LayerKvWriteBatchItem const& item = batch.items[i];
            if (!item.status.ok()) continue;
            auto* t = dynamic_cast<HipTokenTransaction*>(batchBackend(item));
            if (t == nullptr || t->owner_.get() != owner_.get() || t->stream_ != stream_) {
                TokenTransactionBackend::writeLayerBatch(batch);
                return;
            }
            lanes.push_back(t);
            index.push_back(i);
        }
        // Each lane's job is held for the layer's attention launch, which
        // stores the token (its reads take the token from the job's rows:
        // one launch per layer).
        bool any = false;
        for (std::size_t k = 0; k < lanes.size(); ++k) {
            LayerKvWriteBatchItem& item = batch.items[index[k]];
            kimkv_append_job job{};
            HipStatus const s = lanes[k]->prepareWrite(item.write, job);
            if (!s.ok()) {
                item.status = mapDevice(s);
                continue;
            }
            lanes[k]->holdWrite(job);
            item.status = {};
            any = true;
        }
        if (any) owner_->batched_write_submissions.fetch_add(1, std::memory_order_relaxed);
    }

    EngineKvStatus commit(EngineStream) override
    {
        HipStatus const done = finish();
        if (!done.ok()) return mapDevice(done);
        std::lock_guard<std::mutex> lock(owner_->mutex);
        KvCacheError const c = owner_->manager.commitTokenReservation(reservation_);
        if (c != KvCacheError::None) return mapMetadata(c);
        auto it = owner_->requests.find(request_);
        if (it == owner_->requests.end()) return {EngineKvError::InternalError};
        ++it->second.length;
        // The device copy holds the candidate, which is now the committed table.
        if (it->second.table.ptr == table_) it->second.table.version = committed_version_ + 1;
        --owner_->active_transactions;
        resolved_ = true;
        return {};
    }

    void rollback(EngineStream) noexcept override
    {
        if (resolved_) return;
        static_cast<void>(finish());
        std::lock_guard<std::mutex> lock(owner_->mutex);
        static_cast<void>(owner_->manager.rollbackTokenReservation(reservation_));
        if (owner_->active_transactions != 0) --owner_->active_transactions;
        resolved_ = true;
    }

private:
    bool collect(PagedDecodeBatch& batch, std::vector<HipTokenTransaction*>& lanes, std::vector<std::size_t>& index)
    {
        for (std::size_t i = 0; i < batch.item_count; ++i) {
            PagedDecodeBatchItem const& item = batch.items[i];
            if (!item.status.ok()) continue;
            auto* t = dynamic_cast<HipTokenTransaction*>(batchBackend(item));
            if (t == nullptr || t->owner_.get() != owner_.get() || t->stream_ != stream_) return false;
            lanes.push_back(t);
            index.push_back(i);
        }
        return true;
    }

    HipStatus failSubmission(int native) noexcept
    {
        submission_ = HipStatus{HipError::SubmissionFailed, native};
        return submission_;
    }

    HipStatus prepareWrite(LayerKvWrite const& write, kimkv_append_job& job)
    {
        if (finished_ || !submission_.ok() || write.layer >= owner_->config.kv_layout.layer_count
            || write.device_key == nullptr || write.device_value == nullptr) {
            return !submission_.ok() ? submission_ : invalidArgument();
        }
        if (owner_->storage.consumeFailure(HipFailurePoint::Submission)) {
            submission_ = injectedSubmission();
            return submission_;
        }
        job.src_key = write.device_key;
        job.src_value = write.device_value;
        job.src_layer_stride = 0;
        job.src_token_stride = 0;
        job.layer_begin = write.layer;
        job.layer_count = 1;
        job.token_count = 1;
        job.dst_slot = tail_.slot;
        job.dst_kind = static_cast<std::uint8_t>(tail_.kind);
        job.dst_token = tail_token_;
        if (cow_tokens_ != 0) {
            job.cow_slot = cow_src_.slot;
            job.cow_kind = static_cast<std::uint8_t>(cow_src_.kind);
            job.cow_tokens = cow_tokens_;
        }
        return {};
    }

    // A layer's token write is not launched on its own: writeLayer checks it
    // and holds the job, and the layer's attention launch
    // (kimkv_paged_decode_write_batch or _lanes) stores the token, reading
    // the positions it writes from the job's rows and copy-on-write source
    // rather than from the page.  The state machine admits attendLayer(l) only after writeLayer(l)
    // and commit only after every layer's attention, so a held job is either
    // written by its attention launch or dropped with a rollback.
    void holdWrite(kimkv_append_job const& job) noexcept
    {
        held_write_ = job;
        holding_ = true;
    }

    kimkv_append_job takeWrite() noexcept
    {
        kimkv_append_job job{};   // token_count 0: nothing to write
        if (holding_) job = held_write_;
        holding_ = false;
        return job;
    }

    HipStatus checkAttention(PagedDecodeRequest const& r)
    {
        if (finished_ || !submission_.ok() || r.layer >= owner_->config.kv_layout.layer_count
            || r.device_query == nullptr || r.device_output == nullptr || r.device_workspace == nullptr
            || !(r.attention_scale > 0.0F)) {
            return !submission_.ok() ? submission_ : invalidArgument();
        }
        if (token_count_ == 0) return invalidArgument();
        if (owner_->storage.consumeFailure(HipFailurePoint::Submission)) {
            submission_ = injectedSubmission();
            return submission_;
        }
        return {};
    }

    DevicePagedDecodeBatchItem deviceItem(PagedDecodeRequest const& r, bool uses_workspace) const
    {
        return DevicePagedDecodeBatchItem{reinterpret_cast<DeviceBlockDescriptor const*>(descriptors_), desc_count_,
                                          token_count_, r.layer, r.device_query,
                                          uses_workspace ? static_cast<float*>(r.device_workspace) : nullptr,
                                          r.device_output, r.attention_scale};
    }

    HipStatus planOne(PagedDecodeRequest const& r, kimkv_decode_item& item, std::vector<std::uint32_t>& prefix,
                      std::uint32_t& chunk, std::uint32_t& total)
    {
        HipStatus const s = checkAttention(r);
        if (!s.ok()) return s;
        std::uint32_t const QH = owner_->config.query_head_count;
        if (kimkv_decode_plan(owner_->storage.handle(), &token_count_, 1, QH, &chunk, prefix.data(), &total)
            != KIMKV_OK) {
            return invalidArgument();
        }
        std::size_t const need =
            kimkv_decode_workspace_bytes(token_count_, chunk, QH, owner_->config.kv_layout.head_dimension);
        if (r.workspace_bytes < need) return invalidArgument();
        DevicePagedDecodeBatchItem const d = deviceItem(r, need != 0);
        static_assert(sizeof(d) == sizeof(item));
        std::memcpy(&item, &d, sizeof(item));
        return {};
    }

    HipStatus finish() noexcept
    {
        if (finished_) return final_;
        if (!submission_.ok()) {
            static_cast<void>(kimkv_stream_synchronize(stream_));
            final_ = submission_;
        } else {
            // The last attention launch carries a mark; anything enqueued after
            // it (a rollback mid-layer) is drained with the whole stream.
            kimkv_status const waited = mark_ != nullptr && !dirty_ ? kimkv_event_synchronize(mark_->event)
                                                                     : kimkv_stream_synchronize(stream_);
            if (waited != KIMKV_OK) {
                final_ = HipStatus{HipError::ExecutionFailed, kimkv_last_native_error()};
            } else if (owner_->storage.consumeFailure(HipFailurePoint::Completion)) {
                final_ = HipStatus{HipError::ExecutionFailed, -1};
            } else {
                final_ = {};
            }
        }
        finished_ = true;
        mark_.reset();
        releaseDescriptors();
        return final_;
    }

    void setMark(std::shared_ptr<CompletionMark> mark) noexcept
    {
        if (mark == nullptr) return;   // keep dirty: finish() drains the stream instead
        mark_ = std::move(mark);
        dirty_ = false;
    }

    void releaseDescriptors() noexcept { descriptors_ = nullptr; }

    std::shared_ptr<BackendState> owner_;
    KvTokenReservationId reservation_;
    RequestId request_;
    std::uint64_t committed_version_;
    HipStream stream_;
    std::uint32_t token_count_;
    PageHandle tail_{};
    std::uint16_t tail_token_{0};
    PageHandle cow_src_{};
    std::uint16_t cow_tokens_{0};
    kimkv_append_job held_write_{};
    bool holding_{false};
    kimkv_block_desc const* table_{nullptr};         // the request's device table
    kimkv_block_desc const* descriptors_{nullptr};   // table_ until the transaction finishes
    std::uint32_t desc_count_{0};
    std::shared_ptr<CompletionMark> mark_;
    bool dirty_{false};   // work enqueued after mark_ (or no mark yet)
    HipStatus submission_{HipError::InvalidArgument, 0};
    HipStatus final_{};
    bool finished_{false};
    bool resolved_{false};
};

}  // namespace

// ---- chunked prefill ------------------------------------------------------------

struct PrefillChunk::Impl {
    std::shared_ptr<BackendState> owner;
    RequestId request{kInvalidRequestId};
    std::uint32_t begin{0};
    std::uint32_t count{0};
    HipStream stream{nullptr};
    PageLeaseId lease_before{kInvalidPageLeaseId};
    PageLeaseId lease_after{kInvalidPageLeaseId};
    std::shared_ptr<DescriptorArena> arena;
    kimkv_block_desc const* descriptors{nullptr};
    std::uint32_t desc_count{0};
    std::vector<kimkv_append_job> jobs;       // per-layer template: destinations and COW source
    std::vector<std::uint32_t> offsets;       // each job's first token relative to `begin`
    std::uint32_t next_layer{0};
    bool wrote{false};
    HipStatus submission{};
    bool finished{false};
    EngineKvStatus final_status{};
    std::shared_ptr<CompletionMark> mark;
    bool dirty{true};

    ~Impl() { static_cast<void>(finish()); }

    EngineKvStatus check(std::uint32_t layer, bool want_written) const
    {
        if (finished) return {EngineKvError::InvalidState};
        if (!submission.ok()) return mapDevice(submission);
        if (layer != next_layer || wrote != want_written) return {EngineKvError::LayerOutOfOrder};
        return {};
    }

    // Appends this chunk's layer jobs (sources set) to `out`.
    void layerJobs(std::uint32_t layer, KvScalar const* key, KvScalar const* value,
                   std::vector<kimkv_append_job>& out) const
    {
        std::size_t const hd = static_cast<std::size_t>(owner->config.kv_layout.kv_head_count)
            * owner->config.kv_layout.head_dimension;
        for (std::size_t k = 0; k < jobs.size(); ++k) {
            kimkv_append_job j = jobs[k];
            std::size_t const off = static_cast<std::size_t>(offsets[k]) * hd;
            j.src_key = key + off;
            j.src_value = value + off;
            j.src_layer_stride = 0;
            j.src_token_stride = static_cast<std::uint32_t>(hd);
            j.layer_begin = layer;
            j.layer_count = 1;
            out.push_back(j);
        }
    }

    kimkv_prefill_item item(std::uint32_t layer, KvScalar const* query, KvScalar* output, float scale) const
    {
        kimkv_prefill_item it{};
        it.descriptors = descriptors;
        it.descriptor_count = desc_count;
        it.token_count = begin + count;
        it.new_tokens = count;
        it.layer = layer;
        it.query = query;
        it.output = output;
        it.attention_scale = scale;
        return it;
    }

    void fail(int native) { submission = HipStatus{HipError::SubmissionFailed, native}; }

    EngineKvStatus finish()
    {
        if (finished || owner == nullptr) return final_status;
        kimkv_status waited = KIMKV_OK;
        if (!submission.ok()) {
            static_cast<void>(kimkv_stream_synchronize(stream));
        } else {
            waited = mark != nullptr && !dirty ? kimkv_event_synchronize(mark->event) : kimkv_stream_synchronize(stream);
        }
        bool const all_layers = next_layer == owner->config.kv_layout.layer_count;
        if (!submission.ok()) {
            final_status = mapDevice(submission);
        } else if (waited != KIMKV_OK) {
            final_status = {EngineKvError::ExecutionFailed};
        } else if (owner->storage.consumeFailure(HipFailurePoint::Completion)) {
            final_status = {EngineKvError::ExecutionFailed};
        } else if (!all_layers) {
            final_status = {EngineKvError::InvalidState};   // abandoned before its last layer
        } else {
            final_status = {};
        }
        {
            std::lock_guard<std::mutex> lock(owner->mutex);
            KvCacheManager& m = owner->manager;
            owner->prefilling.erase(request);
            if (lease_after != kInvalidPageLeaseId) static_cast<void>(m.releasePageLease(lease_after));
            if (lease_before != kInvalidPageLeaseId) static_cast<void>(m.releasePageLease(lease_before));
            if (final_status.ok()) {
                auto len = owner->requests.find(request);
                if (len != owner->requests.end()) len->second.length += count;
            } else {
                // The table already names the chunk's pages: cancel rather than expose them.
                static_cast<void>(m.releaseRequest(request));
                owner->requests.erase(request);
            }
        }
        arena.reset();
        mark.reset();
        finished = true;
        return final_status;
    }
};

PrefillChunk::PrefillChunk() noexcept = default;
PrefillChunk::PrefillChunk(std::unique_ptr<Impl> impl) noexcept : impl_(std::move(impl)) {}
PrefillChunk::~PrefillChunk() = default;
PrefillChunk::PrefillChunk(PrefillChunk&&) noexcept = default;
PrefillChunk& PrefillChunk::operator=(PrefillChunk&&) noexcept = default;

std::uint32_t PrefillChunk::tokenBegin() const noexcept { return impl_ ? impl_->begin : 0; }
std::uint32_t PrefillChunk::tokenCount() const noexcept { return impl_ ? impl_->count : 0; }

EngineKvStatus PrefillChunk::writeLayer(std::uint32_t layer, KvScalar const* key, KvScalar const* value)
{
    PrefillChunk* self = this;
    EngineKvStatus st{};
    writePrefillBatch(&self, 1, layer, &key, &value, &st);
    return st;
}

EngineKvStatus PrefillChunk::attendLayer(std::uint32_t layer, KvScalar const* query, KvScalar* output, float scale)
{
    PrefillChunk* self = this;
    EngineKvStatus st{};
    attendPrefillBatch(&self, 1, layer, &query, &output, scale, &st);
    return st;
}

EngineKvStatus PrefillChunk::finish()
{
    if (impl_ == nullptr) return {EngineKvError::InvalidState};
    return impl_->finish();
}

void writePrefillBatch(PrefillChunk* const* chunks, std::size_t count, std::uint32_t layer,
                       KvScalar const* const* keys, KvScalar const* const* values, EngineKvStatus* statuses)
{
    thread_local std::vector<kimkv_append_job> jobs;
    jobs.clear();
    std::vector<PrefillChunk::Impl*> launched;
    BackendState* owner = nullptr;
    HipStream stream = nullptr;
    for (std::size_t i = 0; i < count; ++i) {
        PrefillChunk::Impl* c = chunks[i] != nullptr ? chunks[i]->impl() : nullptr;
        if (c == nullptr) {
            statuses[i] = {EngineKvError::InvalidArgument};
            continue;
        }
        statuses[i] = c->check(layer, false);
        if (!statuses[i].ok()) continue;
        if (keys[i] == nullptr || values[i] == nullptr
            || (owner != nullptr && (c->owner.get() != owner || c->stream != stream))) {
            statuses[i] = {EngineKvError::InvalidArgument};
            continue;
        }
        if (c->owner->storage.consumeFailure(HipFailurePoint::Submission)) {
            c->fail(0);
            statuses[i] = {EngineKvError::SubmissionFailed};
            continue;
        }
        owner = c->owner.get();
        stream = c->stream;
        c->layerJobs(layer, keys[i], values[i], jobs);
        launched.push_back(c);
    }
    if (launched.empty()) return;
    HipKvStorage& st = owner->storage;
    kimkv_status k = KIMKV_SUBMISSION_FAILED;
    {
        std::lock_guard<std::mutex> lock(st.launchMutex());
        void* d = st.ring().stage(jobs.data(), jobs.size() * sizeof(kimkv_append_job), stream);
        if (d != nullptr) {
            k = kimkv_append_batch(st.handle(), static_cast<kimkv_append_job const*>(d),
                                   static_cast<std::uint32_t>(jobs.size()), 1, stream);
        }
    }
    int const native = k == KIMKV_OK ? 0 : kimkv_last_native_error();
    for (std::size_t i = 0; i < count; ++i) {
        PrefillChunk::Impl* c = chunks[i] != nullptr ? chunks[i]->impl() : nullptr;
        if (c == nullptr || std::find(launched.begin(), launched.end(), c) == launched.end()) continue;
        c->dirty = true;
        if (k != KIMKV_OK) {
            c->fail(native);
            statuses[i] = {EngineKvError::SubmissionFailed};
        } else {
            c->wrote = true;
        }
    }
}

void attendPrefillBatch(PrefillChunk* const* chunks, std::size_t count, std::uint32_t layer,
                        KvScalar const* const* queries, KvScalar* const* outputs, float scale,
                        EngineKvStatus* statuses)
{
    thread_local std::vector<kimkv_prefill_item> items;
    items.clear();
    std::vector<PrefillChunk::Impl*> launched;
    BackendState* owner = nullptr;
    HipStream stream = nullptr;
    std::uint32_t per = 0;
    for (std::size_t i = 0; i < count; ++i) {
        PrefillChunk::Impl* c = chunks[i] != nullptr ? chunks[i]->impl() : nullptr;
        if (c == nullptr) {
            statuses[i] = {EngineKvError::InvalidArgument};
            continue;
        }
        statuses[i] = c->check(layer, true);
        if (!statuses[i].ok()) continue;
        // The kernel reads query rows as 16-byte vectors and stores 8-byte output pieces.
        if (queries[i] == nullptr || outputs[i] == nullptr || !(scale > 0.0f)
            || (reinterpret_cast<std::uintptr_t>(queries[i]) & 15u) != 0
            || (reinterpret_cast<std::uintptr_t>(outputs[i]) & 7u) != 0
            || (owner != nullptr && (c->owner.get() != owner || c->stream != stream))) {
            statuses[i] = {EngineKvError::InvalidArgument};
            continue;
        }
        if (c->owner->storage.consumeFailure(HipFailurePoint::Submission)) {
            c->fail(0);
            statuses[i] = {EngineKvError::SubmissionFailed};
            continue;
        }
        if (owner == nullptr) {
            owner = c->owner.get();
            stream = c->stream;
            per = kimkv_prefill_tokens_per_block(owner->storage.handle(), owner->config.query_head_count);
        }
        if (per == 0) {
            statuses[i] = {EngineKvError::InvalidArgument};
            continue;
        }
        items.push_back(c->item(layer, queries[i], outputs[i], scale));
        launched.push_back(c);
    }
    if (launched.empty()) return;
    HipKvStorage& st = owner->storage;
    // Workgroup placement (XCD shares of equal work, heavy blocks beside
    // light ones), planned on the host from the items' token counts.
    thread_local std::vector<std::uint32_t> totals, news;
    thread_local std::vector<kimkv_prefill_block> order;
    totals.clear();
    news.clear();
    for (kimkv_prefill_item const& it : items) {
        totals.push_back(it.token_count);
        news.push_back(it.new_tokens);
    }
    KvLayout const& kl = owner->config.kv_layout;
    kimkv_storage_info info{};
    std::uint32_t const units = kimkv_storage_query(st.handle(), &info) == KIMKV_OK && info.compute_units > 0
        ? static_cast<std::uint32_t>(info.compute_units)
        : 0u;
    auto plan = [&](kimkv_prefill_block* out, std::uint32_t capacity, std::uint32_t* n) {
        return kimkv_prefill_order(kl.kv_head_count, kl.head_dimension, owner->config.query_head_count, units,
                                   totals.data(), news.data(), static_cast<std::uint32_t>(items.size()), out,
                                   capacity, n);
    };
    // The placement depends only on the shape and the items' token counts,
    // which every layer of a step repeats: it is planned again only when
    // they change (tens of microseconds of host time per plan).
    thread_local std::vector<std::uint32_t> plan_key, planned_key;
    plan_key.assign({kl.kv_head_count, kl.head_dimension, owner->config.query_head_count, units});
    plan_key.insert(plan_key.end(), totals.begin(), totals.end());
    plan_key.insert(plan_key.end(), news.begin(), news.end());
    kimkv_status k = KIMKV_OK;
    if (plan_key != planned_key) {
        planned_key.clear();
        std::uint32_t needed = 0;
        k = plan(order.data(), static_cast<std::uint32_t>(order.size()), &needed);
        if (k != KIMKV_OK && needed > order.size()) {
            order.resize(needed);
            k = plan(order.data(), needed, &needed);
        }
        if (k == KIMKV_OK) {
            order.resize(needed);
            planned_key = plan_key;
        }
    }
    std::uint32_t const order_count = static_cast<std::uint32_t>(order.size());
    std::size_t const items_bytes = (items.size() * sizeof(kimkv_prefill_item) + 15) & ~std::size_t{15};
    thread_local std::vector<unsigned char> staging;
    staging.resize(items_bytes + order.size() * sizeof(kimkv_prefill_block));
    std::memcpy(staging.data(), items.data(), items.size() * sizeof(kimkv_prefill_item));
    std::memcpy(staging.data() + items_bytes, order.data(), order.size() * sizeof(kimkv_prefill_block));
    if (k == KIMKV_OK) {
        k = KIMKV_SUBMISSION_FAILED;
        std::lock_guard<std::mutex> lock(st.launchMutex());
        auto* d = static_cast<unsigned char*>(st.ring().stage(staging.data(), staging.size(), stream));
        if (d != nullptr) {
            k = kimkv_paged_prefill_ordered(st.handle(), reinterpret_cast<kimkv_prefill_item const*>(d),
                                            static_cast<std::uint32_t>(items.size()),
                                            reinterpret_cast<kimkv_prefill_block const*>(d + items_bytes),
                                            order_count, owner->config.query_head_count, stream);
        }
        st.ring().fence(stream);
    }
    bool const last = layer + 1 == owner->config.kv_layout.layer_count;
    std::shared_ptr<CompletionMark> mark;
    if (k == KIMKV_OK && last) {
        for (PrefillChunk::Impl* c : launched) {
            mark = markLaunch(c->owner, stream);
            break;
        }
    }
    int const native = k == KIMKV_OK ? 0 : kimkv_last_native_error();
    for (std::size_t i = 0; i < count; ++i) {
        PrefillChunk::Impl* c = chunks[i] != nullptr ? chunks[i]->impl() : nullptr;
        if (c == nullptr || std::find(launched.begin(), launched.end(), c) == launched.end()) continue;
        c->dirty = true;
        if (k != KIMKV_OK) {
            c->fail(native);
            statuses[i] = {EngineKvError::SubmissionFailed};
            continue;
        }
        c->wrote = false;
        ++c->next_layer;
        if (last && mark != nullptr) {
            c->mark = mark;
            c->dirty = false;
        }
    }
}

namespace {

// The descriptor patches of one reserve call.  Patches and their source
// descriptors are staged together in the pinned ring and applied by one
// kimkv_patch_descriptors launch per ring request (the kernel reads the
// staged bytes directly).  Once a launch fails the whole batch has failed.
class PatchBatch final {
public:
    PatchBatch(HipKvStorage& storage, HipStream stream) : storage_(storage), stream_(stream)
    {
        patches_.clear();
        sources_.clear();
    }

    // Queues table[first, first + n) = src[0, n); false once the batch failed.
    bool add(kimkv_block_desc* table, std::uint32_t first, kimkv_block_desc const* src, std::uint32_t n)
    {
        std::size_t const limit = storage_.ring().maxStage();
        while (n != 0 && !failed_) {
            std::size_t const used = bytes(patches_.size() + 1, sources_.size());
            if (used + sizeof(kimkv_block_desc) > limit) {
                if (patches_.empty()) failed_ = true;   // a ring too small for one entry
                else static_cast<void>(flush());
                continue;
            }
            auto const k = static_cast<std::uint32_t>(
                std::min<std::size_t>(n, (limit - used) / sizeof(kimkv_block_desc)));
            patches_.push_back(
                kimkv_descriptor_patch{table, first, k, static_cast<std::uint32_t>(sources_.size()), 0});
            sources_.insert(sources_.end(), src, src + k);
            first += k;
            src += k;
            n -= k;
        }
        return !failed_;
    }

    // Issues what is queued; true when every launch of the batch was issued.
    bool flush()
    {
        if (failed_ || patches_.empty()) return !failed_;
        std::size_t const head = bytes(patches_.size(), 0);
        staging_.resize(bytes(patches_.size(), sources_.size()));
        std::memcpy(staging_.data(), patches_.data(), patches_.size() * sizeof(kimkv_descriptor_patch));
        std::memcpy(staging_.data() + head, sources_.data(), sources_.size() * sizeof(kimkv_block_desc));
        {
            std::lock_guard<std::mutex> launch(storage_.launchMutex());
            storage_.noteDescriptorWrite();
            auto* staged = static_cast<unsigned char*>(storage_.ring().stage(staging_.data(), staging_.size(), stream_));
            kimkv_status const k = staged == nullptr
                ? KIMKV_SUBMISSION_FAILED
                : kimkv_patch_descriptors(reinterpret_cast<kimkv_descriptor_patch const*>(staged),
                                          static_cast<std::uint32_t>(patches_.size()),
                                          reinterpret_cast<kimkv_block_desc const*>(staged + head), stream_);
            storage_.ring().fence(stream_);
            if (k != KIMKV_OK) failed_ = true;
        }
        patches_.clear();
        sources_.clear();
        return !failed_;
    }

private:
    static std::size_t bytes(std::size_t patches, std::size_t sources) noexcept
    {
        return (patches * sizeof(kimkv_descriptor_patch) + 7) / 8 * 8 + sources * sizeof(kimkv_block_desc);
    }

    HipKvStorage& storage_;
    HipStream stream_;
    bool failed_{false};
    static thread_local std::vector<kimkv_descriptor_patch> patches_;
    static thread_local std::vector<kimkv_block_desc> sources_;
    static thread_local std::vector<unsigned char> staging_;
};

thread_local std::vector<kimkv_descriptor_patch> PatchBatch::patches_;
thread_local std::vector<kimkv_block_desc> PatchBatch::sources_;
thread_local std::vector<unsigned char> PatchBatch::staging_;

class HipEngineKvBackend final : public EngineKvBackend {
public:
    explicit HipEngineKvBackend(std::shared_ptr<BackendState> s) : state_(std::move(s)) {}

    EngineKvBackendKind kind() const noexcept override { return EngineKvBackendKind::Heterogeneous; }
    EngineKvConfig config() const noexcept override { return state_->config; }

    EngineKvStatus createRequest(RequestId request_id) override
    {
        std::lock_guard<std::mutex> lock(state_->mutex);
        if (!state_->config.valid() || !state_->storage.status().ok()) return {EngineKvError::InvalidState};
        KvCacheError const e = state_->manager.createRequest(request_id);
        if (e == KvCacheError::None) state_->requests.emplace(request_id, RequestState{});
        return mapMetadata(e);
    }

    EngineKvStatus forkRequest(RequestId source, RequestId child) override
    {
        std::lock_guard<std::mutex> lock(state_->mutex);
        auto it = state_->requests.find(source);
        if (it == state_->requests.end()) return {EngineKvError::RequestNotFound};
        if (state_->prefilling.count(source) != 0) return {EngineKvError::InvalidState};
        KvCacheError const e = state_->manager.forkRequest(source, child);
        if (e == KvCacheError::None) {
            RequestState forked;
            forked.length = it->second.length;
            state_->requests.emplace(child, std::move(forked));
        }
        return mapMetadata(e);
    }

    EngineKvStatus releaseRequest(RequestId request_id) override
    {
        std::lock_guard<std::mutex> lock(state_->mutex);
        if (state_->prefilling.count(request_id) != 0) return {EngineKvError::InvalidState};
        KvCacheError const e = state_->manager.releaseRequest(request_id);
        if (e == KvCacheError::None) state_->requests.erase(request_id);
        return mapMetadata(e);
    }

    TokenReserveResult reserveToken(ReserveTokenRequest const& request) override
    {
        TokenReserveResult result;
        reserveBatch(&request, 1, &result);
        return result;
    }

    // Chunk records for a batched attention of the reserved transactions in
    // reservation order (the usual next call), queued into the reserve
    // call's patch launch: that attention then launches from device lane
    // records without a copy of its own.  An attention of other lanes or in
    // another order misses them and copies its own.  At most
    // KIMKV_DECODE_ARG_PREFIX_LANES lanes; nullptr when nothing was queued.
    template <typename Pending>
    BackendState::LaneRecords* seedLaneRecords(std::vector<Pending> const& pending, HipStream stream,
                                               PatchBatch& patches)
    {
        std::size_t const n = pending.size();
        if (n == 0 || n > KIMKV_DECODE_ARG_PREFIX_LANES) return nullptr;
        HipKvStorage& st = state_->storage;
        std::uint32_t const QH = state_->config.query_head_count;
        thread_local std::vector<std::uint32_t> tokens;
        thread_local std::vector<std::uint32_t> pre;
        thread_local std::vector<kimkv_decode_lane> lanes;
        tokens.resize(n);
        pre.assign(n + 1, 0);
        lanes.resize(n);
        for (std::size_t i = 0; i < n; ++i) {
            tokens[i] = pending[i].tx->tokenCount();
            lanes[i] = pending[i].tx->plannedLaneRecord(pending[i].table->ptr, pending[i].r.entry_count);
        }
        std::uint32_t chunk = 0;
        std::uint32_t total = 0;
        if (kimkv_decode_plan(st.handle(), tokens.data(), static_cast<std::uint32_t>(n), QH, &chunk, pre.data(),
                              &total) != KIMKV_OK
            || (chunk & KIMKV_DECODE_GUIDED) != 0) {
            return nullptr;
        }
        thread_local std::vector<unsigned char> key;
        thread_local std::vector<kimkv_block_desc> blob;
        laneRecordKey(lanes, pre, chunk, key);
        if (!expandLaneRecords(key, total, blob)) return nullptr;
        BackendState::LaneRecords* e = nullptr;
        kimkv_block_desc* dst = nullptr;
        {
            std::lock_guard<std::mutex> launch(st.launchMutex());
            e = state_->seedLaneRecords(key, blob.size() * sizeof(kimkv_block_desc), stream);
            if (e != nullptr) dst = static_cast<kimkv_block_desc*>(e->device.get());
        }
        if (e == nullptr) return nullptr;
        // No launch can name these records before this call returns its
        // transactions; the patch batch takes the launch mutex itself.  The
        // patch kernel copies each patch with one workgroup, a word per
        // thread per round trip to the staged (host) bytes, so the records
        // go in pieces of one round each, copied side by side.
        constexpr std::uint32_t kPiece = 256 / 5;   // descriptors: 5 words each
        bool queued = true;
        for (std::uint32_t k = 0; queued && k < blob.size(); k += kPiece) {
            std::uint32_t const m = std::min<std::uint32_t>(kPiece, static_cast<std::uint32_t>(blob.size()) - k);
            queued = patches.add(dst, k, blob.data() + k, m);
        }
        if (!queued) {
            std::lock_guard<std::mutex> launch(st.launchMutex());
            e->key.clear();
            return nullptr;
        }
        return e;
    }

    // reserveToken for several requests sharing one stream.  Per request:
    // the manager's delta reservation, the new tail entry checked, and the
    // request's device table brought to the candidate -- its tail entry
    // patched, or the whole table written when the device copy is stale or
    // too small.  The patches of the call go to the device in one launch.  A
    // request that fails keeps its own status and does not affect the others.
    void reserveBatch(ReserveTokenRequest const* requests, std::size_t count, TokenReserveResult* results)
    {
        std::lock_guard<std::mutex> lock(state_->mutex);
        KvCacheManager& m = state_->manager;
        HipKvStorage& st = state_->storage;
        struct Pending {
            std::size_t index;
            TokenReservationDelta r;
            std::unique_ptr<HipTokenTransaction> tx;
            DeviceTable* table;
        };
        std::vector<Pending> pending;
        pending.reserve(count);
        HipStream const stream = count != 0 ? requests[0].stream : nullptr;
        PatchBatch patches(st, stream);
        thread_local std::vector<kimkv_block_desc> whole;
        for (std::size_t i = 0; i < count; ++i) {
            ReserveTokenRequest const& request = requests[i];
            TokenReserveResult& result = results[i];
            result = TokenReserveResult{};
            if (request.request_id == kInvalidRequestId || request.stream != stream) {
                result.status = {EngineKvError::InvalidArgument};
                continue;
            }
            auto rs = state_->requests.find(request.request_id);
            if (rs == state_->requests.end()) {
                result.status = {EngineKvError::RequestNotFound};
                continue;
            }
            if (state_->prefilling.count(request.request_id) != 0) {
                result.status = {EngineKvError::InvalidState};
                continue;
            }
            TokenReservationDelta const r = m.reserveTokenDelta(request.request_id, request.expected_committed_tokens);
            if (!r.ok()) {
                result.status = mapMetadata(r.error);
                continue;
            }
            DeviceTable& table = rs->second.table;
            bool const rewrite = table.version != r.committed_version || table.capacity() < r.entry_count;
            kimkv_block_desc tail{};
            EngineKvStatus refuse{};
            if (!st.status().ok()) {
                refuse = mapDevice(st.status());
            } else if (!st.descriptor(r.tail, tail)) {
                refuse = {EngineKvError::InvalidArgument};
            } else if (rewrite) {
                // The committed table is checked whole once, when written whole.
                table.version = kStaleTable;
                std::optional<BlockTable> committed = m.blockTable(request.request_id);
                if (!committed || committed->version() != r.committed_version || !st.validTable(*committed)
                    || committed->entries().size() + (r.appended ? 1 : 0) != r.entry_count) {
                    refuse = {EngineKvError::InvalidArgument};
                } else {
                    st.descriptors(*committed, whole);
                    if (r.appended) {
                        whole.push_back(tail);
                    } else {
                        whole.back() = tail;
                    }
                }
            }
            if (refuse.ok() && st.consumeFailure(HipFailurePoint::Submission)) {
                refuse = {EngineKvError::SubmissionFailed};
            }
            if (refuse.ok() && rewrite && !table.fit(st.buffers(), r.entry_count)) {
                refuse = {EngineKvError::ResourceExhausted};
            }
            std::unique_ptr<HipTokenTransaction> tx;
            if (refuse.ok()) {
                try {
                    tx = std::make_unique<HipTokenTransaction>(state_, r, stream);
                } catch (...) {
                    refuse = {EngineKvError::ResourceExhausted};
                }
            }
            if (refuse.ok()) {
                table.version = kStaleTable;   // holds the candidate from here on
                bool const queued = rewrite ? patches.add(table.ptr, 0, whole.data(), r.entry_count)
                                            : patches.add(table.ptr, r.entry_count - 1, &tail, 1);
                if (!queued) refuse = {EngineKvError::SubmissionFailed};
            }
            if (!refuse.ok()) {
                tx.reset();   // drains the stream (patches of this call may be in flight)
                static_cast<void>(m.rollbackTokenReservation(r.reservation_id));
                result.status = refuse;
                continue;
            }
            pending.push_back(Pending{i, r, std::move(tx), &table});
        }
        if (pending.empty()) return;
        BackendState::LaneRecords* seeded = seedLaneRecords(pending, stream, patches);
        bool const issued = patches.flush();
        if (!issued && seeded != nullptr) {
            std::lock_guard<std::mutex> launch(st.launchMutex());
            seeded->key.clear();   // the copy was not issued
        }
        for (Pending& p : pending) {
            TokenReserveResult& result = results[p.index];
            if (!issued) {
                p.tx.reset();   // drains its stream before the metadata is undone
                static_cast<void>(m.rollbackTokenReservation(p.r.reservation_id));
                result.status = {EngineKvError::SubmissionFailed};
                continue;
            }
            p.tx->attach(p.table->ptr, p.r.entry_count);
            std::uint64_t const id = state_->next_transaction_id.fetch_add(1, std::memory_order_relaxed);
            result.transaction = TokenTransaction(std::move(p.tx), id, p.r.request_id, p.r.logical_token_position,
                                                  state_->config.kv_layout.layer_count, stream);
            if (!result.transaction.valid()) {
                result.status = {EngineKvError::InternalError};
                continue;
            }
            ++state_->active_transactions;
            result.status = {};
        }
    }

    EngineKvBackendSnapshot snapshot() const override
    {
        std::lock_guard<std::mutex> lock(state_->mutex);
        EngineKvBackendSnapshot s;
        s.request_count = state_->requests.size();
        s.active_transaction_count = state_->active_transactions;
        for (auto const& kv : state_->requests) s.committed_token_count += kv.second.length;
        s.batched_attention_submissions = state_->batched_attention_submissions.load(std::memory_order_relaxed);
        s.batched_attention_lanes = state_->batched_attention_lanes.load(std::memory_order_relaxed);
        s.batched_write_submissions = state_->batched_write_submissions.load(std::memory_order_relaxed);
        s.storage_reserved_bytes = state_->storage.snapshot().totalReservedBytes();
        KvCacheManagerSnapshot const m = state_->manager.snapshot();
        s.primary_page_tokens = kMicroPageTokenCapacity;
        s.secondary_page_tokens = kExtentPageTokenCapacity;
        s.primary_page_capacity = m.micro_pool.total_slots;
        s.secondary_page_capacity = m.extent_pool.total_slots;
        s.allocated_primary_pages = m.micro_pool.allocated_slots;
        s.allocated_secondary_pages = m.extent_pool.allocated_slots;
        s.successful_primary_allocations = m.micro_pool.successful_allocations;
        s.successful_secondary_allocations = m.extent_pool.successful_allocations;
        s.failed_primary_allocations = m.micro_pool.failed_allocations;
        s.failed_secondary_allocations = m.extent_pool.failed_allocations;
        return s;
    }

    bool checkInvariants() const override
    {
        std::lock_guard<std::mutex> lock(state_->mutex);
        return state_->config.valid() && state_->storage.status().ok() && state_->manager.checkInvariants()
            && state_->active_transactions == state_->manager.snapshot().token_reservation_count;
    }

    // Promotes every run of 8 full sealed micro pages of a committed request.
    // The manager serialises promotions of one request (a commit is checked
    // against the table version seen at prepare), so the metadata goes run by
    // run: prepare, IO lease, release, commit.  The copies are then issued as
    // one batched launch and waited for, all under the backend lock: this
    // backend is the only user of its manager, so no source page freed by a
    // commit can be handed out again before the copy has read it, and no
    // reader can reserve the request before its extents hold the data.  A
    // failed copy cancels the request (its table already names the extents).
    EngineKvStatus promote(RequestId request_id, HipStream stream, std::uint32_t* promoted)
    {
        if (promoted) *promoted = 0;
        std::lock_guard<std::mutex> lock(state_->mutex);
        KvCacheManager& m = state_->manager;
        std::optional<BlockTable> t = m.blockTable(request_id);
        if (!t.has_value()) return {EngineKvError::RequestNotFound};
        if (state_->prefilling.count(request_id) != 0) return {EngineKvError::InvalidState};
        std::vector<std::uint32_t> runs;
        auto const& e = t->entries();
        for (std::size_t i = 0; i + kPromotionSourcePageCount <= e.size();) {
            bool run = true;
            for (std::size_t k = 0; k < kPromotionSourcePageCount && run; ++k) {
                run = e[i + k].kind == PageKind::Micro && e[i + k].valid_tokens == kMicroPageTokenCapacity;
            }
            if (run) {
                runs.push_back(e[i].logical_token_begin);
                i += kPromotionSourcePageCount;
            } else {
                ++i;
            }
        }
        std::vector<PromotionPrepareResult> committed;
        EngineKvStatus status{};
        for (std::uint32_t begin : runs) {
            PromotionPrepareResult p = m.preparePromotion(request_id, begin);
            if (!p.ok()) {
                if (p.error == KvCacheError::RequestConflict || p.error == KvCacheError::ResourceExhausted) break;
                continue;   // not eligible (e.g. a shared or still-mutable page): leave the run as micro
            }
            PageLeaseAcquireResult l = m.acquirePromotionIoLease(p.promotion_id);
            if (!l.ok()) {
                static_cast<void>(m.rollbackPromotion(p.promotion_id));
                status = mapMetadata(l.error);
                break;
            }
            static_cast<void>(m.releasePageLease(l.lease_id));
            KvCacheError const c = m.commitPromotion(p.promotion_id);
            if (c != KvCacheError::None) {
                status = mapMetadata(c);
                break;
            }
            committed.push_back(p);
        }
        if (committed.empty()) return status;
        HipStatus const copied = state_->storage.promoteBatch(committed, stream);
        if (!copied.ok()) {
            static_cast<void>(m.releaseRequest(request_id));
            state_->requests.erase(request_id);
            return mapDevice(copied);
        }
        if (promoted) *promoted = static_cast<std::uint32_t>(committed.size());
        return status;
    }

    // Bulk append of prompt KV ([layer][K/V][token_count][head][dim]) to a
    // request with no token in flight: one metadata append, one batched
    // append launch (waited for), then the full tail is sealed and, when
    // asked, every complete 64-token run is promoted.  A device failure
    // cancels the request, as HipKvCache::append does.
    EngineKvStatus appendPrefill(RequestId request_id, std::uint32_t token_count, KvScalar const* device_kv,
                                 HipStream stream, bool promote_runs, std::uint32_t* promoted)
    {
        if (promoted) *promoted = 0;
        if (request_id == kInvalidRequestId || token_count == 0 || device_kv == nullptr) {
            return {EngineKvError::InvalidArgument};
        }
        PageLeaseAcquireResult before;
        PageLeaseAcquireResult after;
        std::uint32_t begin = 0;
        {
            std::lock_guard<std::mutex> lock(state_->mutex);
            if (!state_->storage.status().ok()) return mapDevice(state_->storage.status());
            auto len = state_->requests.find(request_id);
            if (len == state_->requests.end()) return {EngineKvError::RequestNotFound};
            if (state_->prefilling.count(request_id) != 0) return {EngineKvError::InvalidState};
            KvCacheManager& m = state_->manager;
            before = m.acquireRequestReadLease(request_id);
            if (!before.ok()) return mapMetadata(before.error);
            begin = before.table.tokenCount();
            KvCacheError const appended = m.append(request_id, token_count);
            if (appended != KvCacheError::None) {
                static_cast<void>(m.releasePageLease(before.lease_id));
                return mapMetadata(appended);
            }
            after = m.acquireRequestReadLease(request_id);
            if (!after.ok()) {
                static_cast<void>(m.releasePageLease(before.lease_id));
                static_cast<void>(m.releaseRequest(request_id));
                state_->requests.erase(request_id);
                return mapMetadata(after.error);
            }
        }
        HipStatus const device =
            state_->storage.append(before.table, after.table, begin, token_count, device_kv, stream);
        {
            std::lock_guard<std::mutex> lock(state_->mutex);
            KvCacheManager& m = state_->manager;
            static_cast<void>(m.releasePageLease(after.lease_id));
            static_cast<void>(m.releasePageLease(before.lease_id));
            if (!device.ok()) {
                static_cast<void>(m.releaseRequest(request_id));
                state_->requests.erase(request_id);
                return mapDevice(device);
            }
            auto len = state_->requests.find(request_id);
            if (len == state_->requests.end()) return {EngineKvError::RequestNotFound};
            len->second.length += token_count;
            MappingEntry const& tail = after.table.entries().back();
            if (tail.valid_tokens == kMicroPageTokenCapacity && tail.kind == PageKind::Micro) {
                KvCacheError const sealed = m.sealTail(request_id);
                if (sealed != KvCacheError::None) return mapMetadata(sealed);
            }
        }
        return promote_runs ? promote(request_id, stream, promoted) : EngineKvStatus{};
    }

    PrefillChunkResult beginPrefill(RequestId request_id, std::uint32_t expected, std::uint32_t n, HipStream stream)
    {
        PrefillChunkResult result;
        if (request_id == kInvalidRequestId || n == 0) {
            result.status = {EngineKvError::InvalidArgument};
            return result;
        }
        auto impl = std::make_unique<PrefillChunk::Impl>();
        std::lock_guard<std::mutex> lock(state_->mutex);
        HipKvStorage& st = state_->storage;
        KvCacheManager& m = state_->manager;
        if (!st.status().ok()) {
            result.status = mapDevice(st.status());
            return result;
        }
        auto len = state_->requests.find(request_id);
        if (len == state_->requests.end()) {
            result.status = {EngineKvError::RequestNotFound};
            return result;
        }
        if (len->second.length != expected || state_->prefilling.count(request_id) != 0) {
            result.status = {EngineKvError::InvalidState};
            return result;
        }
        PageLeaseAcquireResult before = m.acquireRequestReadLease(request_id);
        if (!before.ok()) {
            result.status = mapMetadata(before.error);
            return result;
        }
        if (before.table.tokenCount() != expected) {
            static_cast<void>(m.releasePageLease(before.lease_id));
            result.status = {EngineKvError::InvalidState};
            return result;
        }
        KvCacheError const appended = m.append(request_id, n);
        if (appended != KvCacheError::None) {
            static_cast<void>(m.releasePageLease(before.lease_id));
            result.status = mapMetadata(appended);
            return result;
        }
        PageLeaseAcquireResult after = m.acquireRequestReadLease(request_id);
        auto cancel = [&](EngineKvStatus why) {
            if (after.ok()) static_cast<void>(m.releasePageLease(after.lease_id));
            static_cast<void>(m.releasePageLease(before.lease_id));
            static_cast<void>(m.releaseRequest(request_id));
            state_->requests.erase(request_id);
            result.status = why;
            return std::move(result);
        };
        if (!after.ok()) return cancel(mapMetadata(after.error));
        if (!st.appendSegments(before.table, after.table, expected, n, impl->jobs, impl->offsets)) {
            return cancel({EngineKvError::InvalidArgument});
        }
        if (st.consumeFailure(HipFailurePoint::Submission)) return cancel({EngineKvError::SubmissionFailed});
        std::vector<kimkv_block_desc> d;
        st.descriptors(after.table, d);
        std::size_t const bytes = d.size() * sizeof(kimkv_block_desc);
        std::size_t granted = 0;
        void* mem = st.buffers().acquire(bytes, granted);
        if (mem == nullptr) return cancel({EngineKvError::ResourceExhausted});
        try {
            impl->arena = std::make_shared<DescriptorArena>(state_, mem, granted);
        } catch (...) {
            st.buffers().release(mem, granted);
            return cancel({EngineKvError::ResourceExhausted});
        }
        {
            // Fenced by the chunk's first attention launch on this stream.
            std::lock_guard<std::mutex> launch(st.launchMutex());
            st.noteDescriptorWrite();
            if (!st.ring().uploadTo(impl->arena->ptr, d.data(), bytes, stream)) {
                return cancel({EngineKvError::SubmissionFailed});
            }
        }
        state_->prefilling.insert(request_id);
        impl->owner = state_;
        impl->request = request_id;
        impl->begin = expected;
        impl->count = n;
        impl->stream = stream;
        impl->lease_before = before.lease_id;
        impl->lease_after = after.lease_id;
        impl->descriptors = static_cast<kimkv_block_desc const*>(impl->arena->ptr);
        impl->desc_count = static_cast<std::uint32_t>(d.size());
        result.chunk = PrefillChunk(std::move(impl));
        result.status = {};
        return result;
    }

    // Shuffles a pool's free list with a seeded permutation (benchmarks: page
    // ids scattered over the pool).  Only while no request exists.
    EngineKvStatus permuteFreeSlots(PageKind kind, std::uint64_t seed)
    {
        std::lock_guard<std::mutex> lock(state_->mutex);
        if (!state_->requests.empty()) return {EngineKvError::InvalidState};
        return mapMetadata(permuteFreeSlotsOf(state_->manager, kind, seed));
    }

    std::shared_ptr<BackendState> const& state() const noexcept { return state_; }

private:
    std::shared_ptr<BackendState> state_;
};

}  // namespace

std::unique_ptr<EngineKvBackend> createHeterogeneousHipEngineKvBackend(EngineKvConfig config,
                                                                       std::uint32_t micro_page_capacity,
                                                                       std::uint32_t extent_page_capacity)
{
    if (!config.valid() || micro_page_capacity == 0 || extent_page_capacity == 0) return nullptr;
    try {
        auto state = std::make_shared<BackendState>(config, micro_page_capacity, extent_page_capacity);
        if (!state->storage.status().ok()) return nullptr;
        return std::make_unique<HipEngineKvBackend>(std::move(state));
    } catch (...) {
        return nullptr;
    }
}

bool injectHipEngineFailureOnce(EngineKvBackend& backend, HipFailurePoint point) noexcept
{
    auto* b = dynamic_cast<HipEngineKvBackend*>(&backend);
    if (b == nullptr) return false;
    b->state()->storage.injectFailureOnce(point);
    return true;
}

EngineKvStatus promoteRequest(EngineKvBackend& backend, RequestId request_id, HipStream stream,
                              std::uint32_t* promoted_pages)
{
    auto* b = dynamic_cast<HipEngineKvBackend*>(&backend);
    if (b == nullptr) return {EngineKvError::InvalidArgument};
    return b->promote(request_id, stream, promoted_pages);
}

bool engineBlockTable(EngineKvBackend const& backend, RequestId request_id, BlockTable& out)
{
    auto const* b = dynamic_cast<HipEngineKvBackend const*>(&backend);
    if (b == nullptr) return false;
    std::optional<BlockTable> t = b->state()->manager.blockTable(request_id);
    if (!t.has_value()) return false;
    out = std::move(*t);
    return true;
}

EngineKvStatus appendPrefill(EngineKvBackend& backend, RequestId request_id, std::uint32_t token_count,
                             KvScalar const* device_kv, HipStream stream, bool promote_runs,
                             std::uint32_t* promoted_pages)
{
    auto* b = dynamic_cast<HipEngineKvBackend*>(&backend);
    if (b == nullptr) return {EngineKvError::InvalidArgument};
    return b->appendPrefill(request_id, token_count, device_kv, stream, promote_runs, promoted_pages);
}

bool reserveTokenBatch(EngineKvBackend& backend, ReserveTokenRequest const* requests, std::size_t count,
                       TokenReserveResult* results)
{
    auto* b = dynamic_cast<HipEngineKvBackend*>(&backend);
    if (b == nullptr) return false;
    b->reserveBatch(requests, count, results);
    return true;
}

PrefillChunkResult beginPrefillChunk(EngineKvBackend& backend, RequestId request_id, std::uint32_t expected,
                                     std::uint32_t token_count, HipStream stream)
{
    auto* b = dynamic_cast<HipEngineKvBackend*>(&backend);
    if (b == nullptr) {
        PrefillChunkResult r;
        r.status = {EngineKvError::InvalidArgument};
        return r;
    }
    return b->beginPrefill(request_id, expected, token_count, stream);
}

EngineKvStatus permuteEngineFreeSlots(EngineKvBackend& backend, PageKind kind, std::uint64_t seed)
{
    auto* b = dynamic_cast<HipEngineKvBackend*>(&backend);
    if (b == nullptr) return {EngineKvError::InvalidArgument};
    return b->permuteFreeSlots(kind, seed);
}

void const* engineStorage(EngineKvBackend const& backend) noexcept
{
    auto const* b = dynamic_cast<HipEngineKvBackend const*>(&backend);
    return b != nullptr ? b->state()->storage.handle() : nullptr;
}

std::uint64_t laneRecordLaunches(EngineKvBackend const& backend) noexcept
{
    auto const* b = dynamic_cast<HipEngineKvBackend const*>(&backend);
    return b != nullptr ? b->state()->lane_record_launches.load(std::memory_order_relaxed) : 0;
}

}  // namespace kimkvcache
