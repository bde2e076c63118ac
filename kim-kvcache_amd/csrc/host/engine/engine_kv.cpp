// TokenTransaction: the per-token state machine of the engine SPI, and the
// ragged batch entry points over it.
//
// Contract (include/kim-kv/engine/engine_kv.h; reference semantics in
// src/engine/engine_kv.cpp:9-318): a token advances layer by layer, write
// then attend; a call that is not admitted returns its error and submits
// nothing; a submitted step that fails leaves the token Failed (only
// rollback remains); commit is the single completion point; an abandoned
// token rolls back.  Batch lanes are admitted one by one, the first admitted
// lane's backend submits the whole batch once, and each lane settles on its
// own status.
//
// The phase table this file implements:
//
//   phase                   admitted step      success ->                        failure ->
//   AwaitingLayerWrite      Write(next_layer)  AwaitingLayerAttention            Failed
//   AwaitingLayerAttention  Attend(next_layer) AwaitingLayerWrite of next layer, Failed
//                                              or ReadyToCommit after the last
//   ReadyToCommit           commit             Committed                         RolledBack
//   any live phase          rollback           RolledBack
#include "kim-kv/engine/engine_kv.h"

#include <utility>

namespace kimkvcache {
namespace {

constexpr EngineKvStatus fail(EngineKvError e) noexcept { return EngineKvStatus{e}; }

constexpr bool live(TokenTransactionPhase p) noexcept
{
    return p == TokenTransactionPhase::AwaitingLayerWrite || p == TokenTransactionPhase::AwaitingLayerAttention
        || p == TokenTransactionPhase::ReadyToCommit || p == TokenTransactionPhase::Failed;
}

bool writeArgumentsOk(LayerKvWrite const& w) noexcept { return w.device_key != nullptr && w.device_value != nullptr; }

bool attendArgumentsOk(PagedDecodeRequest const& r) noexcept
{
    return r.device_query != nullptr && r.device_output != nullptr && r.device_workspace != nullptr
        && r.workspace_bytes != 0 && r.attention_scale > 0.0F;
}

// Per-item access for the two batch kinds.
std::uint32_t layerOf(PagedDecodeBatchItem const& item) noexcept { return item.request.layer; }
std::uint32_t layerOf(LayerKvWriteBatchItem const& item) noexcept { return item.write.layer; }
bool argumentsOk(PagedDecodeBatchItem const& item) noexcept { return attendArgumentsOk(item.request); }
bool argumentsOk(LayerKvWriteBatchItem const& item) noexcept { return writeArgumentsOk(item.write); }

}  // namespace

// ---- TokenTransactionBackend defaults ---------------------------------------------------------------------

namespace {

// Runs `one(backend, item, stream)` for every item that is still ok.
template <typename Item, typename One>
void eachLane(Item* items, std::size_t count, One one)
{
    for (std::size_t i = 0; i < count; ++i) {
        Item& item = items[i];
        if (!item.status.ok()) continue;
        TokenTransactionBackend* b = item.transaction != nullptr ? one.backendOf(item) : nullptr;
        item.status = b == nullptr ? fail(EngineKvError::InvalidState) : one(*b, item);
    }
}

}  // namespace

void TokenTransactionBackend::attendLayerBatch(PagedDecodeBatch& batch)
{
    struct One {
        TokenTransactionBackend* backendOf(PagedDecodeBatchItem const& i) const noexcept { return batchBackend(i); }
        EngineKvStatus operator()(TokenTransactionBackend& b, PagedDecodeBatchItem const& i) const
        {
            return b.attendLayer(i.request, batchStream(i));
        }
    };
    eachLane(batch.items, batch.item_count, One{});
}

void TokenTransactionBackend::writeLayerBatch(LayerKvWriteBatch& batch)
{
    struct One {
        TokenTransactionBackend* backendOf(LayerKvWriteBatchItem const& i) const noexcept { return batchBackend(i); }
        EngineKvStatus operator()(TokenTransactionBackend& b, LayerKvWriteBatchItem const& i) const
        {
            return b.writeLayer(i.write, batchStream(i));
        }
    };
    eachLane(batch.items, batch.item_count, One{});
}

TokenTransactionBackend* TokenTransactionBackend::batchBackend(PagedDecodeBatchItem const& item) noexcept
{
    return item.transaction == nullptr ? nullptr : item.transaction->backend_.get();
}

EngineStream TokenTransactionBackend::batchStream(PagedDecodeBatchItem const& item) noexcept
{
    return item.transaction == nullptr ? nullptr : item.transaction->stream_;
}

TokenTransactionBackend* TokenTransactionBackend::batchBackend(LayerKvWriteBatchItem const& item) noexcept
{
    return item.transaction == nullptr ? nullptr : item.transaction->backend_.get();
}

EngineStream TokenTransactionBackend::batchStream(LayerKvWriteBatchItem const& item) noexcept
{
    return item.transaction == nullptr ? nullptr : item.transaction->stream_;
}

// ---- TokenTransaction -------------------------------------------------------------------------------------

TokenTransaction::TokenTransaction(std::unique_ptr<TokenTransactionBackend> backend, TokenTransactionId transaction_id,
                                   RequestId request_id, std::uint32_t logical_token_position,
                                   std::uint32_t layer_count, EngineStream stream) noexcept
{
    bool const usable = backend != nullptr && transaction_id != kInvalidTokenTransactionId
        && request_id != kInvalidRequestId && layer_count != 0;
    if (!usable) {
        // A backend handed over with unusable identifiers is released at once.
        if (backend != nullptr) backend->rollback(stream);
        return;
    }
    backend_ = std::move(backend);
    transaction_id_ = transaction_id;
    request_id_ = request_id;
    logical_token_position_ = logical_token_position;
    layer_count_ = layer_count;
    stream_ = stream;
    phase_ = TokenTransactionPhase::AwaitingLayerWrite;
}

TokenTransaction::~TokenTransaction() { rollbackNoexcept(); }

TokenTransaction::TokenTransaction(TokenTransaction&& other) noexcept { adopt(other); }

TokenTransaction& TokenTransaction::operator=(TokenTransaction&& other) noexcept
{
    if (this != &other) {
        rollbackNoexcept();   // an uncommitted token being replaced rolls back
        adopt(other);
    }
    return *this;
}

void TokenTransaction::adopt(TokenTransaction& other) noexcept
{
    backend_ = std::move(other.backend_);
    transaction_id_ = std::exchange(other.transaction_id_, kInvalidTokenTransactionId);
    request_id_ = std::exchange(other.request_id_, kInvalidRequestId);
    logical_token_position_ = std::exchange(other.logical_token_position_, 0u);
    layer_count_ = std::exchange(other.layer_count_, 0u);
    next_layer_ = std::exchange(other.next_layer_, 0u);
    phase_ = std::exchange(other.phase_, TokenTransactionPhase::Empty);
    stream_ = std::exchange(other.stream_, nullptr);
}

bool TokenTransaction::active() const noexcept { return backend_ != nullptr && live(phase_); }

bool TokenTransaction::valid() const noexcept { return active(); }

TokenTransactionSnapshot TokenTransaction::snapshot() const noexcept
{
    TokenTransactionSnapshot s;
    s.transaction_id = transaction_id_;
    s.request_id = request_id_;
    s.logical_token_position = logical_token_position_;
    s.layer_count = layer_count_;
    s.next_layer = next_layer_;
    s.phase = phase_;
    return s;
}

EngineKvStatus TokenTransaction::admit(Step step, std::uint32_t layer, bool arguments_ok) const noexcept
{
    if (!active()) return fail(EngineKvError::InvalidState);
    TokenTransactionPhase const expected =
        step == Step::Write ? TokenTransactionPhase::AwaitingLayerWrite : TokenTransactionPhase::AwaitingLayerAttention;
    if (phase_ != expected || layer != next_layer_) return fail(EngineKvError::LayerOutOfOrder);
    if (!arguments_ok) return fail(EngineKvError::InvalidArgument);
    return {};
}

void TokenTransaction::settle(Step step, EngineKvStatus const& outcome) noexcept
{
    if (!outcome.ok()) {
        phase_ = TokenTransactionPhase::Failed;
    } else if (step == Step::Write) {
        phase_ = TokenTransactionPhase::AwaitingLayerAttention;
    } else {
        ++next_layer_;
        phase_ = next_layer_ < layer_count_ ? TokenTransactionPhase::AwaitingLayerWrite
                                            : TokenTransactionPhase::ReadyToCommit;
    }
}

void TokenTransaction::end(TokenTransactionPhase final_phase) noexcept
{
    backend_.reset();
    phase_ = final_phase;
}

EngineKvStatus TokenTransaction::writeLayer(LayerKvWrite const& write)
{
    EngineKvStatus const admitted = admit(Step::Write, write.layer, writeArgumentsOk(write));
    if (!admitted.ok()) return admitted;
    EngineKvStatus const outcome = backend_->writeLayer(write, stream_);
    settle(Step::Write, outcome);
    return outcome;
}

EngineKvStatus TokenTransaction::attendLayer(PagedDecodeRequest const& request)
{
    EngineKvStatus const admitted = admit(Step::Attend, request.layer, attendArgumentsOk(request));
    if (!admitted.ok()) return admitted;
    EngineKvStatus const outcome = backend_->attendLayer(request, stream_);
    settle(Step::Attend, outcome);
    return outcome;
}

EngineKvStatus TokenTransaction::commit()
{
    if (!active() || phase_ != TokenTransactionPhase::ReadyToCommit) return fail(EngineKvError::InvalidState);
    EngineKvStatus const outcome = backend_->commit(stream_);
    if (!outcome.ok()) backend_->rollback(stream_);   // a token that cannot complete is undone
    end(outcome.ok() ? TokenTransactionPhase::Committed : TokenTransactionPhase::RolledBack);
    return outcome;
}

EngineKvStatus TokenTransaction::rollback() noexcept
{
    if (!active()) return fail(EngineKvError::InvalidState);
    rollbackNoexcept();
    return {};
}

void TokenTransaction::rollbackNoexcept() noexcept
{
    if (!active()) return;
    backend_->rollback(stream_);
    end(TokenTransactionPhase::RolledBack);
}

// ---- batches ----------------------------------------------------------------------------------------------

// Admission, one submission and per-lane settling, shared by both batch kinds.
struct TokenBatchRunner {
    template <typename Item, typename Submit>
    static void run(Item* items, std::size_t count, TokenTransaction::Step step, bool batch_ok, Submit submit)
    {
        if (items == nullptr || count == 0) return;
        TokenTransactionBackend* submitter = nullptr;
        for (std::size_t i = 0; i < count; ++i) {
            Item& item = items[i];
            TokenTransaction const* t = item.transaction;
            item.dispatched = false;
            if (!batch_ok) {
                item.status = fail(EngineKvError::InvalidArgument);
            } else if (t == nullptr) {
                item.status = fail(EngineKvError::InvalidState);
            } else {
                item.status = t->admit(step, layerOf(item), argumentsOk(item));
            }
            if (!item.status.ok()) continue;
            item.dispatched = true;
            if (submitter == nullptr) submitter = t->backend_.get();
        }
        if (submitter == nullptr) return;
        submit(*submitter);
        for (std::size_t i = 0; i < count; ++i) {
            Item& item = items[i];
            TokenTransaction* t = item.transaction;
            // A transaction listed twice settles once: the second entry no longer admits.
            if (item.dispatched && t != nullptr && t->admit(step, layerOf(item), true).ok()) {
                t->settle(step, item.status);
            }
        }
    }

    static void attend(PagedDecodeBatch& batch)
    {
        // The caller's item scratch must hold every lane (reference contract).
        bool const scratch_ok = batch.host_items != nullptr && batch.device_items != nullptr
            && batch.item_capacity >= batch.item_count;
        run(batch.items, batch.item_count, TokenTransaction::Step::Attend, scratch_ok,
            [&batch](TokenTransactionBackend& b) { b.attendLayerBatch(batch); });
    }

    static void write(LayerKvWriteBatch& batch)
    {
        run(batch.items, batch.item_count, TokenTransaction::Step::Write, true,
            [&batch](TokenTransactionBackend& b) { b.writeLayerBatch(batch); });
    }
};

void attendLayerBatch(PagedDecodeBatch& batch) { TokenBatchRunner::attend(batch); }

void writeLayerBatch(LayerKvWriteBatch& batch) { TokenBatchRunner::write(batch); }

}  // namespace kimkvcache
