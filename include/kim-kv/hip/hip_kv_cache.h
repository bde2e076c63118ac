// Micro-benchmark facade over the manager and the device pools; counterpart
// of the reference's include/kim-kv/cuda/cuda_kv_cache.h:33-100.  Every
// operation is submitted on the given stream and waited for before returning;
// the manager's mutex is not held while waiting.
#pragma once

#include "kim-kv/core/kv_layout.h"
#include "kim-kv/hip/hip_status.h"
#include "kim-kv/runtime/kv_cache_manager.h"

#include <cstdint>
#include <memory>
#include <optional>

namespace kimkvcache {

class HipKvStorage;

struct HipKvOperationResult final {
    KvCacheError metadata_error{KvCacheError::None};
    HipStatus device_status{};

    [[nodiscard]] constexpr bool ok() const noexcept { return metadata_error == KvCacheError::None && device_status.ok(); }
    [[nodiscard]] explicit constexpr operator bool() const noexcept { return ok(); }
};

class HipKvCache final {
public:
    HipKvCache(KvLayout layout, std::uint32_t micro_capacity, std::uint32_t extent_capacity);
    ~HipKvCache();

    HipKvCache(HipKvCache const&) = delete;
    HipKvCache& operator=(HipKvCache const&) = delete;

    [[nodiscard]] HipStatus status() const noexcept;
    [[nodiscard]] KvCacheError createRequest(RequestId request_id);
    [[nodiscard]] KvCacheError sealTail(RequestId request_id);
    [[nodiscard]] KvCacheError forkRequest(RequestId source_request_id, RequestId child_request_id);
    [[nodiscard]] KvCacheError releaseRequest(RequestId request_id);

    // device_input: [layer][K/V][token_count][head][dim].  A device failure
    // after the metadata append cancels the request.
    [[nodiscard]] HipKvOperationResult append(RequestId request_id, std::uint32_t token_count,
                                              KvScalar const* device_input, HipStream stream = nullptr);
    // append for `count` requests with one kernel launch (no reference
    // counterpart: the reference appends request by request).  results[i] is
    // what append(request_ids[i], token_count, device_inputs[i]) would
    // return; a device failure cancels every request whose metadata was
    // appended in this call.
    void appendBatch(RequestId const* request_ids, std::size_t count, std::uint32_t token_count,
                     KvScalar const* const* device_inputs, HipStream stream, HipKvOperationResult* results);
    [[nodiscard]] HipKvOperationResult promote(RequestId request_id, std::uint32_t logical_token_begin,
                                               HipStream stream = nullptr);
    // device_output: [layer][K/V][tokens][head][dim].
    [[nodiscard]] HipKvOperationResult gather(RequestId request_id, KvScalar* device_output,
                                              HipStream stream = nullptr);
    // Contiguous MHA reference attention with fp32 query/output [layer][head][dim].
    [[nodiscard]] HipKvOperationResult referenceAttention(RequestId request_id, float const* device_query,
                                                          float* device_output, HipStream stream = nullptr);

    [[nodiscard]] std::optional<BlockTable> blockTable(RequestId request_id) const;
    [[nodiscard]] KvCacheManagerSnapshot metadataSnapshot() const;
    [[nodiscard]] HipStorageSnapshot storageSnapshot() const noexcept;
    [[nodiscard]] bool checkInvariants() const;
    void injectFailureOnce(HipFailurePoint point) noexcept;

    KvCacheManager& manager() noexcept { return manager_; }
    [[nodiscard]] void const* storageHandle() const noexcept;

private:
    KvCacheManager manager_;
    std::unique_ptr<HipKvStorage> storage_;
};

}  // namespace kimkvcache
