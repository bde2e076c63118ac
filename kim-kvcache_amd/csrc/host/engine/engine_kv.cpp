// TokenTransaction state machine and the ragged batch entry points
// (semantics of src/engine/engine_kv.cpp:9-318 in the reference: argument
// errors never submit, a failed call moves the token to Failed, commit is the
// only completion point, and batch lanes succeed or fail independently).
#include "kim-kv/engine/engine_kv.h"

#include <utility>

namespace kimkvcache {
namespace {

constexpr EngineKvStatus status(EngineKvError e) noexcept { return EngineKvStatus{e}; }

bool decodeArgumentsValid(PagedDecodeRequest const& r) noexcept
{
    return r.device_query != nullptr && r.device_output != nullptr && r.device_workspace != nullptr
        && r.workspace_bytes != 0 && r.attention_scale > 0.0F;
}

}  // namespace

TokenTransactionBackend* TokenTransactionBackend::batchBackend(PagedDecodeBatchItem const& item) noexcept
{
    return item.transaction != nullptr ? item.transaction->backend_.get() : nullptr;
}

EngineStream TokenTransactionBackend::batchStream(PagedDecodeBatchItem const& item) noexcept
{
    return item.transaction != nullptr ? item.transaction->stream_ : nullptr;
}

TokenTransactionBackend* TokenTransactionBackend::batchBackend(LayerKvWriteBatchItem const& item) noexcept
{
    return item.transaction != nullptr ? item.transaction->backend_.get() : nullptr;
}

EngineStream TokenTransactionBackend::batchStream(LayerKvWriteBatchItem const& item) noexcept
{
    return item.transaction != nullptr ? item.transaction->stream_ : nullptr;
}

void TokenTransactionBackend::attendLayerBatch(PagedDecodeBatch& batch)
{
    for (std::size_t i = 0; i < batch.item_count; ++i) {
        PagedDecodeBatchItem& item = batch.items[i];
        if (!item.status.ok()) continue;
        TokenTransactionBackend* b = batchBackend(item);
        item.status = b == nullptr ? status(EngineKvError::InvalidState) : b->attendLayer(item.request, batchStream(item));
    }
}

void TokenTransactionBackend::writeLayerBatch(LayerKvWriteBatch& batch)
{
    for (std::size_t i = 0; i < batch.item_count; ++i) {
        LayerKvWriteBatchItem& item = batch.items[i];
        if (!item.status.ok()) continue;
        TokenTransactionBackend* b = batchBackend(item);
        item.status = b == nullptr ? status(EngineKvError::InvalidState) : b->writeLayer(item.write, batchStream(item));
    }
}

TokenTransaction::TokenTransaction(std::unique_ptr<TokenTransactionBackend> backend, TokenTransactionId transaction_id,
                                   RequestId request_id, std::uint32_t logical_token_position,
                                   std::uint32_t layer_count, EngineStream stream) noexcept
    : backend_(std::move(backend)),
      transaction_id_(transaction_id),
      request_id_(request_id),
      logical_token_position_(logical_token_position),
      layer_count_(layer_count),
      phase_(TokenTransactionPhase::AwaitingLayerWrite),
      stream_(stream)
{
    if (backend_ == nullptr || transaction_id_ == kInvalidTokenTransactionId || request_id_ == kInvalidRequestId
        || layer_count_ == 0) {
        if (backend_ != nullptr) backend_->rollback(stream_);
        backend_.reset();
        resetMovedFrom();
    }
}

TokenTransaction::~TokenTransaction() { rollbackNoexcept(); }

TokenTransaction::TokenTransaction(TokenTransaction&& other) noexcept
    : backend_(std::move(other.backend_)),
      transaction_id_(other.transaction_id_),
      request_id_(other.request_id_),
      logical_token_position_(other.logical_token_position_),
      layer_count_(other.layer_count_),
      next_layer_(other.next_layer_),
      phase_(other.phase_),
      stream_(other.stream_)
{
    other.resetMovedFrom();
}

TokenTransaction& TokenTransaction::operator=(TokenTransaction&& other) noexcept
{
    if (this == &other) return *this;
    rollbackNoexcept();
    backend_ = std::move(other.backend_);
    transaction_id_ = other.transaction_id_;
    request_id_ = other.request_id_;
    logical_token_position_ = other.logical_token_position_;
    layer_count_ = other.layer_count_;
    next_layer_ = other.next_layer_;
    phase_ = other.phase_;
    stream_ = other.stream_;
    other.resetMovedFrom();
    return *this;
}

bool TokenTransaction::active() const noexcept
{
    switch (phase_) {
    case TokenTransactionPhase::AwaitingLayerWrite:
    case TokenTransactionPhase::AwaitingLayerAttention:
    case TokenTransactionPhase::ReadyToCommit:
    case TokenTransactionPhase::Failed:
        return backend_ != nullptr;
    default:
        return false;
    }
}

bool TokenTransaction::valid() const noexcept { return active(); }

TokenTransactionSnapshot TokenTransaction::snapshot() const noexcept
{
    return TokenTransactionSnapshot{transaction_id_, request_id_, logical_token_position_, layer_count_, next_layer_,
                                    phase_};
}

EngineKvStatus TokenTransaction::writeLayer(LayerKvWrite const& write)
{
    if (!active()) return status(EngineKvError::InvalidState);
    if (phase_ != TokenTransactionPhase::AwaitingLayerWrite || write.layer != next_layer_) {
        return status(EngineKvError::LayerOutOfOrder);
    }
    if (write.device_key == nullptr || write.device_value == nullptr) return status(EngineKvError::InvalidArgument);
    EngineKvStatus const r = backend_->writeLayer(write, stream_);
    if (!r.ok()) {
        phase_ = TokenTransactionPhase::Failed;
        return r;
    }
    phase_ = TokenTransactionPhase::AwaitingLayerAttention;
    return {};
}

void TokenTransaction::advanceAfterAttend() noexcept
{
    ++next_layer_;
    phase_ = next_layer_ == layer_count_ ? TokenTransactionPhase::ReadyToCommit
                                         : TokenTransactionPhase::AwaitingLayerWrite;
}

EngineKvStatus TokenTransaction::attendLayer(PagedDecodeRequest const& request)
{
    if (!active()) return status(EngineKvError::InvalidState);
    if (phase_ != TokenTransactionPhase::AwaitingLayerAttention || request.layer != next_layer_) {
        return status(EngineKvError::LayerOutOfOrder);
    }
    if (!decodeArgumentsValid(request)) return status(EngineKvError::InvalidArgument);
    EngineKvStatus const r = backend_->attendLayer(request, stream_);
    if (!r.ok()) {
        phase_ = TokenTransactionPhase::Failed;
        return r;
    }
    advanceAfterAttend();
    return {};
}

EngineKvStatus TokenTransaction::commit()
{
    if (!active() || phase_ != TokenTransactionPhase::ReadyToCommit) return status(EngineKvError::InvalidState);
    EngineKvStatus const r = backend_->commit(stream_);
    if (!r.ok()) {
        backend_->rollback(stream_);
        backend_.reset();
        phase_ = TokenTransactionPhase::RolledBack;
        return r;
    }
    backend_.reset();
    phase_ = TokenTransactionPhase::Committed;
    return {};
}

EngineKvStatus TokenTransaction::rollback() noexcept
{
    if (!active()) return status(EngineKvError::InvalidState);
    rollbackNoexcept();
    return {};
}

void TokenTransaction::rollbackNoexcept() noexcept
{
    if (!active()) return;
    backend_->rollback(stream_);
    backend_.reset();
    phase_ = TokenTransactionPhase::RolledBack;
}

void TokenTransaction::resetMovedFrom() noexcept
{
    transaction_id_ = kInvalidTokenTransactionId;
    request_id_ = kInvalidRequestId;
    logical_token_position_ = 0;
    layer_count_ = 0;
    next_layer_ = 0;
    phase_ = TokenTransactionPhase::Empty;
    stream_ = nullptr;
}

void attendLayerBatch(PagedDecodeBatch& batch)
{
    if (batch.items == nullptr || batch.item_count == 0) return;
    bool const scratch = batch.host_items != nullptr && batch.device_items != nullptr
        && batch.item_capacity >= batch.item_count;
    TokenTransactionBackend* dispatcher = nullptr;
    for (std::size_t i = 0; i < batch.item_count; ++i) {
        PagedDecodeBatchItem& item = batch.items[i];
        item.status = {};
        item.dispatched = false;
        TokenTransaction* t = item.transaction;
        if (!scratch) {
            item.status = status(EngineKvError::InvalidArgument);
        } else if (t == nullptr || !t->active()) {
            item.status = status(EngineKvError::InvalidState);
        } else if (t->phase_ != TokenTransactionPhase::AwaitingLayerAttention || item.request.layer != t->next_layer_) {
            item.status = status(EngineKvError::LayerOutOfOrder);
        } else if (!decodeArgumentsValid(item.request)) {
            item.status = status(EngineKvError::InvalidArgument);
        } else {
            item.dispatched = true;
            if (dispatcher == nullptr) dispatcher = t->backend_.get();
        }
    }
    if (dispatcher == nullptr) return;
    dispatcher->attendLayerBatch(batch);
    for (std::size_t i = 0; i < batch.item_count; ++i) {
        PagedDecodeBatchItem& item = batch.items[i];
        TokenTransaction* t = item.transaction;
        if (!item.dispatched || t == nullptr || t->phase_ != TokenTransactionPhase::AwaitingLayerAttention
            || item.request.layer != t->next_layer_) {
            continue;
        }
        if (!item.status.ok()) {
            t->phase_ = TokenTransactionPhase::Failed;
            continue;
        }
        t->advanceAfterAttend();
    }
}

void writeLayerBatch(LayerKvWriteBatch& batch)
{
    if (batch.items == nullptr || batch.item_count == 0) return;
    TokenTransactionBackend* dispatcher = nullptr;
    for (std::size_t i = 0; i < batch.item_count; ++i) {
        LayerKvWriteBatchItem& item = batch.items[i];
        item.status = {};
        item.dispatched = false;
        TokenTransaction* t = item.transaction;
        if (t == nullptr || !t->active()) {
            item.status = status(EngineKvError::InvalidState);
        } else if (t->phase_ != TokenTransactionPhase::AwaitingLayerWrite || item.write.layer != t->next_layer_) {
            item.status = status(EngineKvError::LayerOutOfOrder);
        } else if (item.write.device_key == nullptr || item.write.device_value == nullptr) {
            item.status = status(EngineKvError::InvalidArgument);
        } else {
            item.dispatched = true;
            if (dispatcher == nullptr) dispatcher = t->backend_.get();
        }
    }
    if (dispatcher == nullptr) return;
    dispatcher->writeLayerBatch(batch);
    for (std::size_t i = 0; i < batch.item_count; ++i) {
        LayerKvWriteBatchItem& item = batch.items[i];
        TokenTransaction* t = item.transaction;
        if (!item.dispatched || t == nullptr || t->phase_ != TokenTransactionPhase::AwaitingLayerWrite
            || item.write.layer != t->next_layer_) {
            continue;
        }
        t->phase_ = item.status.ok() ? TokenTransactionPhase::AwaitingLayerAttention : TokenTransactionPhase::Failed;
    }
}

}  // namespace kimkvcache
