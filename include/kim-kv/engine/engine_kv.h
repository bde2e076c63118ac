// Narrow KV SPI the model runner sees (include/kim-kv/engine/engine_kv.h of the
// reference): per-token transactions that write each layer's K/V, attend, and
// commit at the token boundary; plus the ragged batch entry points.
//
// Additions over the reference interface (no reference counterpart):
//   * LayerKvWriteBatch / writeLayerBatch: all lanes' writes of one layer in
//     one device launch (the reference launches one kernel per lane).
#pragma once

#include "kim-kv/core/kv_layout.h"
#include "kim-kv/core/page_handle.h"
#include "kim-kv/runtime/promotion.h"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string_view>
#include <type_traits>

namespace kimkvcache {

using EngineStream = void*;
using TokenTransactionId = std::uint64_t;
constexpr TokenTransactionId kInvalidTokenTransactionId = 0;

enum class EngineKvBackendKind : std::uint8_t {
    Heterogeneous,
    Fixed,
};

enum class EngineKvError : std::uint8_t {
    None,
    InvalidArgument,
    InvalidState,
    RequestNotFound,
    RequestAlreadyExists,
    RequestConflict,
    ResourceExhausted,
    LayerOutOfOrder,
    SubmissionFailed,
    ExecutionFailed,
    InternalError,
};

[[nodiscard]] constexpr std::string_view toString(EngineKvError error) noexcept
{
    switch (error) {
    case EngineKvError::None: return "none";
    case EngineKvError::InvalidArgument: return "invalid_argument";
    case EngineKvError::InvalidState: return "invalid_state";
    case EngineKvError::RequestNotFound: return "request_not_found";
    case EngineKvError::RequestAlreadyExists: return "request_already_exists";
    case EngineKvError::RequestConflict: return "request_conflict";
    case EngineKvError::ResourceExhausted: return "resource_exhausted";
    case EngineKvError::LayerOutOfOrder: return "layer_out_of_order";
    case EngineKvError::SubmissionFailed: return "submission_failed";
    case EngineKvError::ExecutionFailed: return "execution_failed";
    case EngineKvError::InternalError: return "internal_error";
    }
    return "unknown";
}

struct EngineKvStatus final {
    EngineKvError error{EngineKvError::None};
    [[nodiscard]] constexpr bool ok() const noexcept { return error == EngineKvError::None; }
    [[nodiscard]] explicit constexpr operator bool() const noexcept { return ok(); }
};

struct EngineKvConfig final {
    KvLayout kv_layout{};
    std::uint32_t query_head_count{0};
    std::size_t attention_workspace_bytes{0};

    [[nodiscard]] constexpr bool valid() const noexcept
    {
        return kv_layout.valid() && query_head_count >= kv_layout.kv_head_count
            && query_head_count % kv_layout.kv_head_count == 0 && attention_workspace_bytes != 0;
    }
};

// Page-table entry as uploaded for the device (20 bytes, same layout as
// kimkv_block_desc in kimkv_hip.h).
struct DeviceBlockDescriptor final {
    std::uint32_t slot{PageHandle::kInvalidSlot};
    std::uint32_t generation{PageHandle::kInvalidGeneration};
    std::uint32_t logical_token_begin{0};
    std::uint16_t valid_tokens{0};
    std::uint16_t page_token_capacity{0};
    PageKind kind{PageKind::Micro};

    [[nodiscard]] constexpr bool valid() const noexcept
    {
        return slot != PageHandle::kInvalidSlot && generation != PageHandle::kInvalidGeneration
            && valid_tokens != 0 && page_token_capacity != 0 && valid_tokens <= page_token_capacity
            && isKnownPageKind(kind);
    }
};
static_assert(std::is_trivially_copyable_v<DeviceBlockDescriptor>);
static_assert(std::is_standard_layout_v<DeviceBlockDescriptor>);
static_assert(sizeof(DeviceBlockDescriptor) == 20);

struct DeviceBlockTableView final {
    DeviceBlockDescriptor const* device_descriptors{nullptr};
    std::uint32_t descriptor_count{0};
    std::uint32_t committed_token_count{0};
    std::uint32_t current_token_position{0};

    [[nodiscard]] constexpr bool valid() const noexcept
    {
        return device_descriptors != nullptr && descriptor_count != 0
            && current_token_position == committed_token_count;
    }
};

// One layer's new K and V for one token: device [kv_heads][head_dim] each.
struct LayerKvWrite final {
    std::uint32_t layer{0};
    KvScalar const* device_key{nullptr};
    KvScalar const* device_value{nullptr};
};

// Decode attention of one token for one layer: device query/output
// [query_heads][head_dim] fp16; `device_workspace` holds split-K partials.
struct PagedDecodeRequest final {
    std::uint32_t layer{0};
    KvScalar const* device_query{nullptr};
    KvScalar* device_output{nullptr};
    void* device_workspace{nullptr};
    std::size_t workspace_bytes{0};
    float attention_scale{0.0F};
};

class TokenTransaction;

// One lane of a ragged decode launch.  `status` is per lane, so one rejected
// or failed lane does not stop the others.
struct PagedDecodeBatchItem final {
    TokenTransaction* transaction{nullptr};
    PagedDecodeRequest request{};
    EngineKvStatus status{EngineKvError::InvalidState};
    bool dispatched{false};
};

// Device-side lane record uploaded once per layer (56 bytes, same layout as
// kimkv_decode_item in kimkv_hip.h).
struct DevicePagedDecodeBatchItem final {
    DeviceBlockDescriptor const* device_descriptors{nullptr};
    std::uint32_t descriptor_count{0};
    std::uint32_t token_count{0};
    std::uint32_t layer{0};
    KvScalar const* device_query{nullptr};
    float* device_scores{nullptr};
    KvScalar* device_output{nullptr};
    float attention_scale{0.0F};
};
static_assert(std::is_trivially_copyable_v<DevicePagedDecodeBatchItem>);
static_assert(std::is_standard_layout_v<DevicePagedDecodeBatchItem>);
static_assert(sizeof(DevicePagedDecodeBatchItem) == 56);

// host_items / device_items: caller-owned scratch with item_capacity entries.
struct PagedDecodeBatch final {
    PagedDecodeBatchItem* items{nullptr};
    std::size_t item_count{0};
    DevicePagedDecodeBatchItem* host_items{nullptr};
    DevicePagedDecodeBatchItem* device_items{nullptr};
    std::size_t item_capacity{0};
};

// Batched writes of one layer (extension): each item is one lane.
struct LayerKvWriteBatchItem final {
    TokenTransaction* transaction{nullptr};
    LayerKvWrite write{};
    EngineKvStatus status{EngineKvError::InvalidState};
    bool dispatched{false};
};

struct LayerKvWriteBatch final {
    LayerKvWriteBatchItem* items{nullptr};
    std::size_t item_count{0};
};

struct ReserveTokenRequest final {
    RequestId request_id{kInvalidRequestId};
    std::uint32_t expected_committed_tokens{0};
    EngineStream stream{nullptr};
};

enum class TokenTransactionPhase : std::uint8_t {
    Empty,
    AwaitingLayerWrite,
    AwaitingLayerAttention,
    ReadyToCommit,
    Failed,
    Committed,
    RolledBack,
};

[[nodiscard]] constexpr std::string_view toString(TokenTransactionPhase phase) noexcept
{
    switch (phase) {
    case TokenTransactionPhase::Empty: return "empty";
    case TokenTransactionPhase::AwaitingLayerWrite: return "awaiting_layer_write";
    case TokenTransactionPhase::AwaitingLayerAttention: return "awaiting_layer_attention";
    case TokenTransactionPhase::ReadyToCommit: return "ready_to_commit";
    case TokenTransactionPhase::Failed: return "failed";
    case TokenTransactionPhase::Committed: return "committed";
    case TokenTransactionPhase::RolledBack: return "rolled_back";
    }
    return "unknown";
}

struct TokenTransactionSnapshot final {
    TokenTransactionId transaction_id{kInvalidTokenTransactionId};
    RequestId request_id{kInvalidRequestId};
    std::uint32_t logical_token_position{0};
    std::uint32_t layer_count{0};
    std::uint32_t next_layer{0};
    TokenTransactionPhase phase{TokenTransactionPhase::Empty};
};

// Backend side of one token.  write/attend only enqueue on the bound stream;
// commit is the single completion checkpoint; rollback waits for in-flight
// device work before releasing metadata.
class TokenTransactionBackend {
public:
    virtual ~TokenTransactionBackend() = default;
    TokenTransactionBackend(TokenTransactionBackend const&) = delete;
    TokenTransactionBackend& operator=(TokenTransactionBackend const&) = delete;

    [[nodiscard]] virtual EngineKvStatus writeLayer(LayerKvWrite const& write, EngineStream stream) = 0;
    [[nodiscard]] virtual EngineKvStatus attendLayer(PagedDecodeRequest const& request, EngineStream stream) = 0;
    // Default: every valid lane on its own.  Device backends override with one launch.
    virtual void attendLayerBatch(PagedDecodeBatch& batch);
    virtual void writeLayerBatch(LayerKvWriteBatch& batch);
    [[nodiscard]] virtual EngineKvStatus commit(EngineStream stream) = 0;
    virtual void rollback(EngineStream stream) noexcept = 0;

protected:
    TokenTransactionBackend() = default;
    [[nodiscard]] static TokenTransactionBackend* batchBackend(PagedDecodeBatchItem const& item) noexcept;
    [[nodiscard]] static EngineStream batchStream(PagedDecodeBatchItem const& item) noexcept;
    [[nodiscard]] static TokenTransactionBackend* batchBackend(LayerKvWriteBatchItem const& item) noexcept;
    [[nodiscard]] static EngineStream batchStream(LayerKvWriteBatchItem const& item) noexcept;
};

// Move-only RAII token: per layer writeLayer -> attendLayer, then commit.
// Destruction or move-assignment over an uncommitted transaction rolls back.
class TokenTransaction final {
public:
    TokenTransaction() noexcept = default;
    TokenTransaction(std::unique_ptr<TokenTransactionBackend> backend, TokenTransactionId transaction_id,
                     RequestId request_id, std::uint32_t logical_token_position, std::uint32_t layer_count,
                     EngineStream stream) noexcept;
    ~TokenTransaction();

    TokenTransaction(TokenTransaction const&) = delete;
    TokenTransaction& operator=(TokenTransaction const&) = delete;
    TokenTransaction(TokenTransaction&& other) noexcept;
    TokenTransaction& operator=(TokenTransaction&& other) noexcept;

    [[nodiscard]] bool valid() const noexcept;
    [[nodiscard]] TokenTransactionSnapshot snapshot() const noexcept;
    [[nodiscard]] EngineKvStatus writeLayer(LayerKvWrite const& write);
    [[nodiscard]] EngineKvStatus attendLayer(PagedDecodeRequest const& request);
    [[nodiscard]] EngineKvStatus commit();
    [[nodiscard]] EngineKvStatus rollback() noexcept;

private:
    // The two per-layer steps of a token.
    enum class Step : std::uint8_t { Write, Attend };

    [[nodiscard]] bool active() const noexcept;
    // Whether `step` for `layer` may be submitted now, as the status the call
    // returns (InvalidState, LayerOutOfOrder, InvalidArgument in that order).
    [[nodiscard]] EngineKvStatus admit(Step step, std::uint32_t layer, bool arguments_ok) const noexcept;
    // Applies a submitted step's outcome: Failed, or the next phase.
    void settle(Step step, EngineKvStatus const& outcome) noexcept;
    void end(TokenTransactionPhase final_phase) noexcept;
    void rollbackNoexcept() noexcept;
    void adopt(TokenTransaction& other) noexcept;

    std::unique_ptr<TokenTransactionBackend> backend_{};
    TokenTransactionId transaction_id_{kInvalidTokenTransactionId};
    RequestId request_id_{kInvalidRequestId};
    std::uint32_t logical_token_position_{0};
    std::uint32_t layer_count_{0};
    std::uint32_t next_layer_{0};
    TokenTransactionPhase phase_{TokenTransactionPhase::Empty};
    EngineStream stream_{nullptr};

    friend class TokenTransactionBackend;
    friend struct TokenBatchRunner;
};

// Validates every lane against its transaction's state machine, dispatches
// the backend batch operation once, then advances or fails lanes separately.
void attendLayerBatch(PagedDecodeBatch& batch);
void writeLayerBatch(LayerKvWriteBatch& batch);

struct TokenReserveResult final {
    EngineKvStatus status{};
    TokenTransaction transaction{};

    [[nodiscard]] bool ok() const noexcept { return status.ok() && transaction.valid(); }
    [[nodiscard]] explicit operator bool() const noexcept { return ok(); }
};

struct EngineKvBackendSnapshot final {
    std::uint64_t request_count{0};
    std::uint64_t active_transaction_count{0};
    std::uint64_t committed_token_count{0};
    std::uint64_t batched_attention_submissions{0};
    std::uint64_t batched_attention_lanes{0};
    std::uint16_t primary_page_tokens{0};
    std::uint16_t secondary_page_tokens{0};
    std::uint32_t primary_page_capacity{0};
    std::uint32_t secondary_page_capacity{0};
    std::uint32_t allocated_primary_pages{0};
    std::uint32_t allocated_secondary_pages{0};
    std::uint64_t successful_primary_allocations{0};
    std::uint64_t successful_secondary_allocations{0};
    std::uint64_t failed_primary_allocations{0};
    std::uint64_t failed_secondary_allocations{0};
    std::uint64_t storage_reserved_bytes{0};
    std::uint64_t batched_write_submissions{0};
};

// The model runner / scheduler depend only on this interface.
class EngineKvBackend {
public:
    virtual ~EngineKvBackend() = default;
    EngineKvBackend(EngineKvBackend const&) = delete;
    EngineKvBackend& operator=(EngineKvBackend const&) = delete;

    [[nodiscard]] virtual EngineKvBackendKind kind() const noexcept = 0;
    [[nodiscard]] virtual EngineKvConfig config() const noexcept = 0;
    [[nodiscard]] virtual EngineKvStatus createRequest(RequestId request_id) = 0;
    [[nodiscard]] virtual EngineKvStatus forkRequest(RequestId source_request_id, RequestId child_request_id) = 0;
    [[nodiscard]] virtual EngineKvStatus releaseRequest(RequestId request_id) = 0;
    [[nodiscard]] virtual TokenReserveResult reserveToken(ReserveTokenRequest const& request) = 0;
    [[nodiscard]] virtual EngineKvBackendSnapshot snapshot() const = 0;
    [[nodiscard]] virtual bool checkInvariants() const = 0;

protected:
    EngineKvBackend() = default;
};

}  // namespace kimkvcache
