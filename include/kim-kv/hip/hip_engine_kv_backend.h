// Factory of the MI355X engine backend; counterpart of the reference's
// include/kim-kv/cuda/cuda_engine_kv_backend.h:11-29.
#pragma once

#include "kim-kv/core/block_table.h"
#include "kim-kv/engine/engine_kv.h"
#include "kim-kv/hip/hip_status.h"

#include <cstdint>
#include <memory>

namespace kimkvcache {

// createHeterogeneousCudaEngineKvBackend: micro (8-token) + extent (64-token)
// device pools; nullptr when the config is invalid or the pools cannot be
// allocated.  Differences: any number of lanes share one decode launch (the
// reference caps the batch at 64), and the attention workspace only has to
// hold the split-K partials (never more than query_heads * tokens * 4 bytes).
[[nodiscard]] std::unique_ptr<EngineKvBackend> createHeterogeneousHipEngineKvBackend(
    EngineKvConfig config, std::uint32_t micro_page_capacity, std::uint32_t extent_page_capacity);

// injectCudaEngineFailureOnce.
[[nodiscard]] bool injectHipEngineFailureOnce(EngineKvBackend& backend, HipFailurePoint point) noexcept;

// Engine-path promotion (no reference counterpart: the reference engine never
// promotes).  Promotes every eligible run of 8 full sealed micro pages of a
// request that has no token in flight, with one batched copy launch on
// `stream`; waits for completion and commits the new tables.
[[nodiscard]] EngineKvStatus promoteRequest(EngineKvBackend& backend, RequestId request_id, HipStream stream,
                                            std::uint32_t* promoted_pages);

// Bulk append of prompt KV, layout [layer][K/V][token_count][head][dim] in
// device memory, to a request with no token in flight (no reference
// counterpart: the reference engine appends one token per transaction).
// Waits for the copy; seals a full tail; with promote_runs, promotes every
// complete run of 8 micro pages as promoteRequest does.  A device failure
// cancels the request.
[[nodiscard]] EngineKvStatus appendPrefill(EngineKvBackend& backend, RequestId request_id,
                                           std::uint32_t token_count, KvScalar const* device_kv, HipStream stream,
                                           bool promote_runs, std::uint32_t* promoted_pages);

// reserveToken for `count` requests on one stream (no reference counterpart:
// the reference reserves lane by lane, with a device allocation and upload
// each).  Results match calling reserveToken in order, except that all
// descriptor tables share one device arena filled by a single upload.  A
// request naming a different stream than requests[0] gets InvalidArgument.
// Returns false when `backend` is not a HIP backend.
[[nodiscard]] bool reserveTokenBatch(EngineKvBackend& backend, ReserveTokenRequest const* requests,
                                     std::size_t count, TokenReserveResult* results);

// Seeded permutation of a pool's free list while no request exists (see
// kim-kv/runtime/pool_permutation.h).
[[nodiscard]] EngineKvStatus permuteEngineFreeSlots(EngineKvBackend& backend, PageKind kind, std::uint64_t seed);

// A chunk of n prompt positions of one request, written and attended layer
// by layer (no reference counterpart: the reference advances a prompt one
// position per token transaction).  beginPrefillChunk appends the n tokens to
// the request's table at once; then, for every layer in order, writeLayer
// stores the chunk's K/V ([n][kv_heads][head_dim] fp16 each) and attendLayer
// runs causal GQA attention of the chunk's queries ([n][query_heads][dim])
// over the request's tokens: output row i equals a decode of the first
// T0 + i + 1 tokens.  finish() waits for the work; a failure cancels the
// request (its table already holds the chunk).  Calls only enqueue work on
// the chunk's stream until finish().
class PrefillChunk final {
public:
    struct Impl;
    PrefillChunk() noexcept;
    explicit PrefillChunk(std::unique_ptr<Impl> impl) noexcept;
    ~PrefillChunk();
    PrefillChunk(PrefillChunk&&) noexcept;
    PrefillChunk& operator=(PrefillChunk&&) noexcept;
    PrefillChunk(PrefillChunk const&) = delete;
    PrefillChunk& operator=(PrefillChunk const&) = delete;

    [[nodiscard]] bool valid() const noexcept { return impl_ != nullptr; }
    [[nodiscard]] std::uint32_t tokenBegin() const noexcept;   // T0
    [[nodiscard]] std::uint32_t tokenCount() const noexcept;   // n
    [[nodiscard]] EngineKvStatus writeLayer(std::uint32_t layer, KvScalar const* device_key,
                                            KvScalar const* device_value);
    [[nodiscard]] EngineKvStatus attendLayer(std::uint32_t layer, KvScalar const* device_query,
                                             KvScalar* device_output, float attention_scale);
    [[nodiscard]] EngineKvStatus finish();
    Impl* impl() noexcept { return impl_.get(); }

private:
    std::unique_ptr<Impl> impl_;
};

struct PrefillChunkResult final {
    EngineKvStatus status{EngineKvError::InternalError};
    PrefillChunk chunk;
    [[nodiscard]] bool ok() const noexcept { return status.ok() && chunk.valid(); }
};

[[nodiscard]] PrefillChunkResult beginPrefillChunk(EngineKvBackend& backend, RequestId request_id,
                                                   std::uint32_t expected_committed_tokens, std::uint32_t token_count,
                                                   HipStream stream);

// The layer step of several chunks of one backend and stream with one launch
// each (write: one append kernel; attend: one prefill kernel).
void writePrefillBatch(PrefillChunk* const* chunks, std::size_t count, std::uint32_t layer,
                       KvScalar const* const* device_keys, KvScalar const* const* device_values,
                       EngineKvStatus* statuses);
void attendPrefillBatch(PrefillChunk* const* chunks, std::size_t count, std::uint32_t layer,
                        KvScalar const* const* device_queries, KvScalar* const* device_outputs, float attention_scale,
                        EngineKvStatus* statuses);

// Committed block table of a request (diagnostics and tests).
[[nodiscard]] bool engineBlockTable(EngineKvBackend const& backend, RequestId request_id, BlockTable& out);

// The backend's device storage handle (kimkv_storage*), for data-path helpers.
[[nodiscard]] void const* engineStorage(EngineKvBackend const& backend) noexcept;

// Batched attention launches that read their lanes from device lane records
// (kimkv_paged_decode_lanes: at most 64 lanes whose per-layer addresses are
// evenly spaced) rather than from items staged in host memory; 0 when
// `backend` is not a HIP backend.  No reference counterpart.
[[nodiscard]] std::uint64_t laneRecordLaunches(EngineKvBackend const& backend) noexcept;

}  // namespace kimkvcache
