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

// Committed block table of a request (diagnostics and tests).
[[nodiscard]] bool engineBlockTable(EngineKvBackend const& backend, RequestId request_id, BlockTable& out);

// The backend's device storage handle (kimkv_storage*), for data-path helpers.
[[nodiscard]] void const* engineStorage(EngineKvBackend const& backend) noexcept;

}  // namespace kimkvcache
