// C facade over the engine backend and HipKvCache (include/kimkv_host.h,
// kimkv_engine_* / kimkv_txn_* / kimkv_cache_*).
#include "kimkv_host.h"

#include "capi_internal.h"
#include "kim-kv/engine/engine_kv.h"
#include "kim-kv/hip/hip_engine_kv_backend.h"
#include "kim-kv/hip/hip_kv_cache.h"

#include <cstring>
#include <memory>
#include <new>
#include <vector>

using namespace kimkvcache;

struct kimkv_txn {
    TokenTransaction t;
};

struct kimkv_prefill_chunk {
    PrefillChunk c;
};

struct kimkv_cache {
    HipKvCache cache;
    kimkv_manager view;
    kimkv_cache(KvLayout l, std::uint32_t micro, std::uint32_t extent) : cache(l, micro, extent)
    {
        view.m = &cache.manager();
    }
};

namespace {

int code(EngineKvStatus s) { return static_cast<int>(s.error); }

int deviceCode(HipStatus s)
{
    switch (s.error) {
    case HipError::None: return KIMKV_OK;
    case HipError::InvalidArgument: return KIMKV_INVALID_ARGUMENT;
    case HipError::RuntimeUnavailable: return KIMKV_RUNTIME_UNAVAILABLE;
    case HipError::AllocationFailed: return KIMKV_ALLOCATION_FAILED;
    case HipError::SubmissionFailed: return KIMKV_SUBMISSION_FAILED;
    case HipError::NotReady: return KIMKV_NOT_READY;
    case HipError::ExecutionFailed: return KIMKV_EXECUTION_FAILED;
    default: return KIMKV_INTERNAL_ERROR;
    }
}

kimkv_cache_result result(HipKvOperationResult r)
{
    return kimkv_cache_result{static_cast<int>(r.metadata_error), deviceCode(r.device_status)};
}

PagedDecodeRequest request(kimkv_decode_request const& r)
{
    return PagedDecodeRequest{r.layer, r.query, r.output, r.workspace, static_cast<std::size_t>(r.workspace_bytes),
                              r.attention_scale};
}

}  // namespace

extern "C" {

kimkv_engine* kimkv_engine_create(const kimkv_engine_config* c, uint32_t micro_capacity, uint32_t extent_capacity)
{
    if (c == nullptr) return nullptr;
    EngineKvConfig config;
    config.kv_layout = KvLayout{c->layers, c->kv_heads, c->head_dim};
    config.query_head_count = c->query_heads;
    config.attention_workspace_bytes = static_cast<std::size_t>(c->attention_workspace_bytes);
    std::unique_ptr<EngineKvBackend> b = createHeterogeneousHipEngineKvBackend(config, micro_capacity, extent_capacity);
    if (b == nullptr) return nullptr;
    auto* e = new (std::nothrow) kimkv_engine{std::move(b)};
    return e;
}

void kimkv_engine_destroy(kimkv_engine* e) { delete e; }

int kimkv_engine_create_request(kimkv_engine* e, uint64_t id) { return code(e->backend->createRequest(id)); }
int kimkv_engine_fork_request(kimkv_engine* e, uint64_t s, uint64_t c) { return code(e->backend->forkRequest(s, c)); }
int kimkv_engine_release_request(kimkv_engine* e, uint64_t id) { return code(e->backend->releaseRequest(id)); }

int kimkv_engine_reserve_token(kimkv_engine* e, uint64_t id, uint32_t expected, kimkv_stream_t stream, kimkv_txn** txn)
{
    if (txn == nullptr) return static_cast<int>(EngineKvError::InvalidArgument);
    *txn = nullptr;
    TokenReserveResult r = e->backend->reserveToken(ReserveTokenRequest{id, expected, stream});
    if (!r.ok()) return r.status.ok() ? static_cast<int>(EngineKvError::InternalError) : code(r.status);
    auto* t = new (std::nothrow) kimkv_txn{std::move(r.transaction)};
    if (t == nullptr) return static_cast<int>(EngineKvError::ResourceExhausted);
    *txn = t;
    return 0;
}

void kimkv_engine_get_snapshot(const kimkv_engine* e, kimkv_engine_snapshot* out)
{
    EngineKvBackendSnapshot const s = e->backend->snapshot();
    out->request_count = s.request_count;
    out->active_transaction_count = s.active_transaction_count;
    out->committed_token_count = s.committed_token_count;
    out->batched_attention_submissions = s.batched_attention_submissions;
    out->batched_attention_lanes = s.batched_attention_lanes;
    out->batched_write_submissions = s.batched_write_submissions;
    out->primary_page_tokens = s.primary_page_tokens;
    out->secondary_page_tokens = s.secondary_page_tokens;
    out->primary_page_capacity = s.primary_page_capacity;
    out->secondary_page_capacity = s.secondary_page_capacity;
    out->allocated_primary_pages = s.allocated_primary_pages;
    out->allocated_secondary_pages = s.allocated_secondary_pages;
    out->successful_primary_allocations = s.successful_primary_allocations;
    out->successful_secondary_allocations = s.successful_secondary_allocations;
    out->failed_primary_allocations = s.failed_primary_allocations;
    out->failed_secondary_allocations = s.failed_secondary_allocations;
    out->storage_reserved_bytes = s.storage_reserved_bytes;
}

int kimkv_engine_check_invariants(const kimkv_engine* e) { return e->backend->checkInvariants() ? 1 : 0; }

int kimkv_engine_inject_failure_once(kimkv_engine* e, uint32_t point)
{
    if (point > 1) return 0;
    return injectHipEngineFailureOnce(*e->backend, point == 0 ? HipFailurePoint::Submission
                                                              : HipFailurePoint::Completion) ? 1 : 0;
}

int kimkv_engine_promote_request(kimkv_engine* e, uint64_t id, kimkv_stream_t stream, uint32_t* promoted)
{
    return code(promoteRequest(*e->backend, id, stream, promoted));
}

int kimkv_engine_block_table(const kimkv_engine* e, uint64_t id, uint64_t* version, kimkv_mapping_entry* entries,
                             uint32_t capacity, uint32_t* count)
{
    BlockTable t;
    if (!engineBlockTable(*e->backend, id, t)) {
        if (count) *count = 0;
        return static_cast<int>(KvCacheError::RequestNotFound);
    }
    auto const& en = t.entries();
    if (version) *version = t.version();
    if (count) *count = static_cast<uint32_t>(en.size());
    if (entries == nullptr) return 0;
    if (en.size() > capacity) return static_cast<int>(KvCacheError::InvalidArgument);
    for (std::size_t i = 0; i < en.size(); ++i) {
        entries[i] = kimkv_mapping_entry{en[i].logical_token_begin, en[i].valid_tokens,
                                         static_cast<uint8_t>(en[i].kind), 0, en[i].handle.slot, en[i].handle.generation};
    }
    return 0;
}

const kimkv_storage* kimkv_engine_storage(const kimkv_engine* e)
{
    return static_cast<const kimkv_storage*>(engineStorage(*e->backend));
}

uint64_t kimkv_engine_lane_record_launches(const kimkv_engine* e)
{
    return laneRecordLaunches(*e->backend);
}

int kimkv_engine_append_prefill(kimkv_engine* e, uint64_t id, uint32_t n, const uint16_t* device_kv,
                                kimkv_stream_t stream, int promote, uint32_t* promoted)
{
    return code(appendPrefill(*e->backend, id, n, device_kv, stream, promote != 0, promoted));
}

int kimkv_engine_permute_free_slots(kimkv_engine* e, uint32_t kind, uint64_t seed)
{
    if (kind > 1) return static_cast<int>(EngineKvError::InvalidArgument);
    return code(permuteEngineFreeSlots(*e->backend, kind == 0 ? PageKind::Micro : PageKind::Extent, seed));
}

void kimkv_engine_reserve_batch(kimkv_engine* e, const uint64_t* ids, const uint32_t* expected, uint32_t count,
                                kimkv_stream_t stream, kimkv_txn** txns, int* statuses)
{
    std::vector<ReserveTokenRequest> requests(count);
    std::vector<TokenReserveResult> results(count);
    for (uint32_t i = 0; i < count; ++i) requests[i] = ReserveTokenRequest{ids[i], expected[i], stream};
    if (!reserveTokenBatch(*e->backend, requests.data(), count, results.data())) {
        for (uint32_t i = 0; i < count; ++i) statuses[i] = kimkv_engine_reserve_token(e, ids[i], expected[i], stream, &txns[i]);
        return;
    }
    for (uint32_t i = 0; i < count; ++i) {
        txns[i] = nullptr;
        TokenReserveResult& r = results[i];
        if (!r.ok()) {
            statuses[i] = r.status.ok() ? static_cast<int>(EngineKvError::InternalError) : code(r.status);
            continue;
        }
        txns[i] = new (std::nothrow) kimkv_txn{std::move(r.transaction)};
        statuses[i] = txns[i] != nullptr ? 0 : static_cast<int>(EngineKvError::ResourceExhausted);
    }
}

int kimkv_txn_write_layer(kimkv_txn* t, uint32_t layer, const uint16_t* key, const uint16_t* value)
{
    return code(t->t.writeLayer(LayerKvWrite{layer, key, value}));
}

int kimkv_txn_attend_layer(kimkv_txn* t, const kimkv_decode_request* r)
{
    if (r == nullptr) return static_cast<int>(EngineKvError::InvalidArgument);
    return code(t->t.attendLayer(request(*r)));
}

int kimkv_txn_commit(kimkv_txn* t) { return code(t->t.commit()); }
int kimkv_txn_rollback(kimkv_txn* t) { return code(t->t.rollback()); }

void kimkv_txn_state(const kimkv_txn* t, uint32_t* phase, uint32_t* next_layer, uint32_t* position)
{
    TokenTransactionSnapshot const s = t->t.snapshot();
    if (phase) *phase = static_cast<uint32_t>(s.phase);
    if (next_layer) *next_layer = s.next_layer;
    if (position) *position = s.logical_token_position;
}

void kimkv_txn_destroy(kimkv_txn* t) { delete t; }

void kimkv_txn_commit_batch(kimkv_txn** txns, uint32_t count, int* statuses)
{
    for (uint32_t i = 0; i < count; ++i) {
        if (txns[i] == nullptr) {
            statuses[i] = static_cast<int>(EngineKvError::InvalidArgument);
            continue;
        }
        statuses[i] = code(txns[i]->t.commit());
        delete txns[i];
        txns[i] = nullptr;
    }
}

void kimkv_attend_layer_batch(kimkv_txn** txns, const kimkv_decode_request* requests, uint32_t count,
                              void* device_items, uint32_t device_capacity, int* statuses)
{
    if (count == 0) return;
    thread_local std::vector<PagedDecodeBatchItem> items;
    thread_local std::vector<DevicePagedDecodeBatchItem> host;
    items.assign(count, PagedDecodeBatchItem{});
    host.resize(count);
    for (uint32_t i = 0; i < count; ++i) {
        items[i].transaction = txns[i] != nullptr ? &txns[i]->t : nullptr;
        items[i].request = request(requests[i]);
    }
    PagedDecodeBatch batch{items.data(), count, host.data(), static_cast<DevicePagedDecodeBatchItem*>(device_items),
                           device_items != nullptr ? device_capacity : 0};
    attendLayerBatch(batch);
    for (uint32_t i = 0; i < count; ++i) statuses[i] = code(items[i].status);
}

void kimkv_write_layer_batch(kimkv_txn** txns, const uint32_t* layers, const uint16_t* const* keys,
                             const uint16_t* const* values, uint32_t count, int* statuses)
{
    if (count == 0) return;
    thread_local std::vector<LayerKvWriteBatchItem> items;
    items.assign(count, LayerKvWriteBatchItem{});
    for (uint32_t i = 0; i < count; ++i) {
        items[i].transaction = txns[i] != nullptr ? &txns[i]->t : nullptr;
        items[i].write = LayerKvWrite{layers[i], keys[i], values[i]};
    }
    LayerKvWriteBatch batch{items.data(), count};
    writeLayerBatch(batch);
    for (uint32_t i = 0; i < count; ++i) statuses[i] = code(items[i].status);
}

int kimkv_engine_prefill_begin(kimkv_engine* e, uint64_t id, uint32_t expected, uint32_t n, kimkv_stream_t stream,
                               kimkv_prefill_chunk** chunk)
{
    if (chunk == nullptr) return static_cast<int>(EngineKvError::InvalidArgument);
    *chunk = nullptr;
    PrefillChunkResult r = beginPrefillChunk(*e->backend, id, expected, n, stream);
    if (!r.ok()) return code(r.status);
    auto* c = new (std::nothrow) kimkv_prefill_chunk{std::move(r.chunk)};
    if (c == nullptr) return static_cast<int>(EngineKvError::ResourceExhausted);   // r.chunk's dtor cancelled it
    *chunk = c;
    return 0;
}

int kimkv_prefill_write_layer(kimkv_prefill_chunk* c, uint32_t layer, const uint16_t* key, const uint16_t* value)
{
    return code(c->c.writeLayer(layer, key, value));
}

int kimkv_prefill_attend_layer(kimkv_prefill_chunk* c, uint32_t layer, const uint16_t* query, uint16_t* output,
                               float attention_scale)
{
    return code(c->c.attendLayer(layer, query, output, attention_scale));
}

int kimkv_prefill_finish(kimkv_prefill_chunk* c) { return code(c->c.finish()); }
void kimkv_prefill_destroy(kimkv_prefill_chunk* c) { delete c; }

void kimkv_prefill_write_batch(kimkv_prefill_chunk** chunks, uint32_t count, uint32_t layer,
                               const uint16_t* const* keys, const uint16_t* const* values, int* statuses)
{
    if (count == 0) return;
    thread_local std::vector<PrefillChunk*> list;
    thread_local std::vector<EngineKvStatus> st;
    list.resize(count);
    st.assign(count, EngineKvStatus{});
    for (uint32_t i = 0; i < count; ++i) list[i] = chunks[i] != nullptr ? &chunks[i]->c : nullptr;
    writePrefillBatch(list.data(), count, layer, keys, values, st.data());
    for (uint32_t i = 0; i < count; ++i) statuses[i] = code(st[i]);
}

void kimkv_prefill_attend_batch(kimkv_prefill_chunk** chunks, uint32_t count, uint32_t layer,
                                const uint16_t* const* queries, uint16_t* const* outputs, float scale, int* statuses)
{
    if (count == 0) return;
    thread_local std::vector<PrefillChunk*> list;
    thread_local std::vector<EngineKvStatus> st;
    list.resize(count);
    st.assign(count, EngineKvStatus{});
    for (uint32_t i = 0; i < count; ++i) list[i] = chunks[i] != nullptr ? &chunks[i]->c : nullptr;
    attendPrefillBatch(list.data(), count, layer, queries, outputs, scale, st.data());
    for (uint32_t i = 0; i < count; ++i) statuses[i] = code(st[i]);
}

kimkv_cache* kimkv_cache_create(kimkv_layout layout, uint32_t micro_capacity, uint32_t extent_capacity)
{
    try {
        return new kimkv_cache(KvLayout{layout.layers, layout.kv_heads, layout.head_dim}, micro_capacity,
                               extent_capacity);
    } catch (...) {
        return nullptr;
    }
}

void kimkv_cache_destroy(kimkv_cache* c) { delete c; }
int kimkv_cache_status(const kimkv_cache* c) { return deviceCode(c->cache.status()); }

kimkv_manager* kimkv_cache_manager(kimkv_cache* c)
{
    return &c->view;
}

const kimkv_storage* kimkv_cache_storage(const kimkv_cache* c)
{
    return static_cast<const kimkv_storage*>(c->cache.storageHandle());
}

kimkv_cache_result kimkv_cache_append(kimkv_cache* c, uint64_t id, uint32_t n, const uint16_t* input,
                                      kimkv_stream_t stream)
{
    return result(c->cache.append(id, n, input, stream));
}

void kimkv_cache_append_batch(kimkv_cache* c, const uint64_t* ids, uint32_t count, uint32_t n,
                              const uint16_t* const* inputs, kimkv_stream_t stream, kimkv_cache_result* out)
{
    std::vector<HipKvOperationResult> results(count);
    c->cache.appendBatch(ids, count, n, inputs, stream, results.data());
    for (uint32_t i = 0; i < count; ++i) out[i] = result(results[i]);
}

kimkv_cache_result kimkv_cache_promote(kimkv_cache* c, uint64_t id, uint32_t begin, kimkv_stream_t stream)
{
    return result(c->cache.promote(id, begin, stream));
}

kimkv_cache_result kimkv_cache_gather(kimkv_cache* c, uint64_t id, uint16_t* out, kimkv_stream_t stream)
{
    return result(c->cache.gather(id, out, stream));
}

kimkv_cache_result kimkv_cache_reference_attention(kimkv_cache* c, uint64_t id, const float* q, float* o,
                                                   kimkv_stream_t stream)
{
    return result(c->cache.referenceAttention(id, q, o, stream));
}

void kimkv_cache_inject_failure_once(kimkv_cache* c, uint32_t point)
{
    c->cache.injectFailureOnce(point == 0 ? HipFailurePoint::Submission : HipFailurePoint::Completion);
}

}  // extern "C"
