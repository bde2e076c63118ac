// Iteration-level FIFO scheduler (src/engine/iteration_scheduler.cpp:1-772 of
// the reference).  Admission gates, per-request state machine, FIFO
// selection of up to max_batched_tokens requests per iteration and the
// per-request quota (prefill_chunk_size prompt positions, one decode
// position) follow the reference.  Execution has two forms:
//   * waves (the reference's): one position of every selected request per
//     model batch, repeated until quotas or the token budget run out;
//   * spans (runners with generationSupportsSpans()): the same positions,
//     distributed round-robin under the budget exactly as the waves would,
//     sent as one call whose prompt chunks are whole spans.
#include "kim-kv/engine/iteration_scheduler.h"

#include "generation_internal.h"

#include <algorithm>
#include <deque>
#include <new>
#include <unordered_map>
#include <utility>

namespace kimkvcache {

class IterationSchedulerRuntime::Impl final {
public:
    struct Record {
        GenerationRequest request{};
        SchedulerRequestState state{SchedulerRequestState::Created};
        GenerationTerminal terminal{};
        detail::RequestProgress progress{};
        std::uint64_t kv_budget{0};
        std::uint32_t prompt_position{0};
        bool cancel_requested{false};

        bool prefilling() const noexcept { return prompt_position < request.prompt_token_ids.size(); }
        bool terminal_state() const noexcept { return state == SchedulerRequestState::Terminal; }
        bool cancelled() const noexcept
        {
            return cancel_requested || (request.cancellation != nullptr && request.cancellation->cancelled());
        }
    };

    // A selected request and the positions it may still take this iteration.
    struct Selected {
        Record* record;
        std::uint32_t quota;
    };

    Impl(EngineKvBackend& k, GenerationModelRunner& r, IterationSchedulerConfig c) noexcept
        : kv(&k), runner(&r), config(c)
    {
    }

    void setState(RequestId id, Record* record, SchedulerRequestState s)
    {
        if (record != nullptr) record->state = s;
        auto it = states.find(id);
        if (it != states.end()) it->second = s;
    }

    SchedulerAdmissionResult reject(RequestId id, SchedulerAdmissionError error, std::string text, bool remember)
    {
        if (remember && id != kInvalidRequestId) {
            try {
                states.emplace(id, SchedulerRequestState::Rejected);
            } catch (std::bad_alloc const&) {
                return {false, SchedulerAdmissionError::InternalError, "rejection bookkeeping allocation failed"};
            }
        }
        return {false, error, std::move(text)};
    }

    void finish(Record& r, GenerationTerminalReason reason, GenerationError error, std::string text)
    {
        if (r.terminal_state()) return;
        detail::completeTerminal(r.terminal, r.progress, *kv, r.request.request_id, reason, error, std::move(text));
        setState(r.request.request_id, &r, SchedulerRequestState::Terminal);
        reserved_kv_tokens -= r.kv_budget;
        try {
            terminals.push_back(r.terminal);
        } catch (std::bad_alloc const&) {
            // Resources are reclaimed; only the delivery copy is lost.
        }
    }

    void stopRecord(Record& r)
    {
        finish(r, GenerationTerminalReason::RuntimeStopped, GenerationError::RuntimeStopped,
               "runtime stopped at an iteration boundary");
    }

    void stopAll()
    {
        while (!queue.empty()) {
            RequestId const id = queue.front();
            queue.pop_front();
            auto it = records.find(id);
            if (it != records.end()) stopRecord(it->second);
        }
    }

    // Boundary checks and lazy KV creation before a request's next position;
    // false when the request ended here.
    bool activate(Record& r)
    {
        if (r.cancelled()) {
            finish(r, GenerationTerminalReason::Cancelled, GenerationError::None,
                   "cancelled at an iteration boundary");
            return false;
        }
        if (stopped.load(std::memory_order_acquire)) {
            stopRecord(r);
            return false;
        }
        if (!r.progress.kv_created) {
            EngineKvStatus const created = kv->createRequest(r.request.request_id);
            if (!created.ok()) {
                finish(r, GenerationTerminalReason::Failed, GenerationError::KvBackendFailed,
                       "KV request creation failed: " + std::string(toString(created.error)));
                return false;
            }
            r.progress.kv_created = true;
            setState(r.request.request_id, &r, SchedulerRequestState::Running);
        }
        return true;
    }

    // The next position of a request: a prompt position while prefilling,
    // else the last emitted token at the position after the prompt.
    static GenerationBatchItem nextItem(Record const& r)
    {
        if (r.prefilling()) {
            return {r.request.request_id, r.request.prompt_token_ids[r.prompt_position], r.prompt_position};
        }
        auto const prompt = static_cast<std::uint32_t>(r.request.prompt_token_ids.size());
        auto const out = static_cast<std::uint32_t>(r.terminal.output_token_ids.size());
        return {r.request.request_id, r.terminal.output_token_ids.back(), prompt + out - 1};
    }

    // Applies the step that followed `positions` positions of the request.
    void advance(Record& r, GenerationStepResult step, std::uint32_t positions, bool prefill)
    {
        if (!step.success) {
            finish(r, GenerationTerminalReason::Failed, GenerationError::ModelFailed, std::move(step.detail));
            return;
        }
        TinyLlamaConfig const model = runner->generationConfig();
        if (step.greedy_token_id >= model.vocabulary_size) {
            finish(r, GenerationTerminalReason::Failed, GenerationError::ModelFailed,
                   "model returned a token id outside the vocabulary");
            return;
        }
        if (prefill) r.prompt_position += positions;
        if (stopped.load(std::memory_order_acquire)) {
            stopRecord(r);
            return;
        }
        if (r.cancelled()) {
            finish(r, GenerationTerminalReason::Cancelled, GenerationError::None,
                   "cancelled at an iteration boundary");
            return;
        }
        if (r.prefilling()) return;
        try {
            r.terminal.output_token_ids.push_back(step.greedy_token_id);
        } catch (std::bad_alloc const&) {
            finish(r, GenerationTerminalReason::Failed, GenerationError::InternalError,
                   "completion token allocation failed");
            return;
        }
        r.progress.tokenEmitted();
        if (step.greedy_token_id == r.request.sampling.eos_token_id.value_or(model.eos_token_id)) {
            finish(r, GenerationTerminalReason::EosToken, GenerationError::None, "EOS token generated");
        } else if (r.terminal.output_token_ids.size() == r.request.sampling.max_new_tokens) {
            finish(r, GenerationTerminalReason::MaxNewTokens, GenerationError::None, "max_new_tokens reached");
        }
    }

    void failAll(std::vector<Selected> const& selected, GenerationError error, char const* text)
    {
        for (Selected const& s : selected) finish(*s.record, GenerationTerminalReason::Failed, error, text);
    }

    void waveIteration(std::vector<Selected>& selected, std::uint32_t budget, std::uint32_t max_batch,
                       SchedulerIterationResult& out)
    {
        struct Planned {
            Record* record;
            GenerationBatchItem item;
            bool prefill;
        };
        std::vector<Planned> plan;
        std::vector<GenerationBatchItem> batch;
        while (budget != 0) {
            plan.clear();
            for (Selected& s : selected) {
                if (s.quota == 0 || budget == 0 || s.record->terminal_state()) continue;
                if (!activate(*s.record)) {
                    s.quota = 0;
                    continue;
                }
                plan.push_back(Planned{s.record, nextItem(*s.record), s.record->prefilling()});
                --s.quota;
                --budget;
            }
            if (plan.empty()) break;
            for (std::size_t b = 0; b < plan.size() && !stopped.load(std::memory_order_acquire); b += max_batch) {
                std::size_t const e = std::min(plan.size(), b + max_batch);
                batch.clear();
                for (std::size_t i = b; i < e; ++i) batch.push_back(plan[i].item);
                GenerationBatchResult r = runner->generationForwardBatch(batch);
                ++out.model_forward_batches;
                out.model_forward_tokens += static_cast<std::uint32_t>(batch.size());
                for (std::size_t i = b; i < e; ++i) (plan[i].prefill ? out.prefill_tokens : out.decode_tokens) += 1;
                if (!r.success || r.steps.size() != batch.size()) {
                    std::string const text = r.detail.empty() ? "model returned an invalid batch result" : r.detail;
                    for (std::size_t i = b; i < e; ++i) {
                        finish(*plan[i].record, GenerationTerminalReason::Failed, GenerationError::ModelFailed, text);
                    }
                    continue;
                }
                for (std::size_t i = b; i < e; ++i) {
                    advance(*plan[i].record, std::move(r.steps[i - b]), 1, plan[i].prefill);
                }
            }
            if (stopped.load(std::memory_order_acquire)) break;
        }
    }

    void spanIteration(std::vector<Selected>& selected, std::uint32_t budget, std::uint32_t max_batch,
                       SchedulerIterationResult& out)
    {
        budget = std::min(budget, max_batch);
        std::vector<Selected*> live;
        for (Selected& s : selected) {
            if (!s.record->terminal_state() && activate(*s.record)) live.push_back(&s);
        }
        // The positions the waves would hand out: one per request per round, FIFO order.
        std::vector<std::uint32_t> take(live.size(), 0);
        for (bool any = true; any && budget != 0;) {
            any = false;
            for (std::size_t i = 0; i < live.size() && budget != 0; ++i) {
                if (take[i] < live[i]->quota) {
                    ++take[i];
                    --budget;
                    any = true;
                }
            }
        }
        std::vector<GenerationSpan> spans;
        std::vector<std::size_t> owner;
        for (std::size_t i = 0; i < live.size(); ++i) {
            if (take[i] == 0) continue;
            Record& r = *live[i]->record;
            GenerationBatchItem const first = nextItem(r);
            GenerationSpan span{r.request.request_id, first.expected_position, {}};
            if (r.prefilling()) {
                auto const b = r.request.prompt_token_ids.begin() + r.prompt_position;
                span.token_ids.assign(b, b + take[i]);
            } else {
                span.token_ids.assign(1, first.token_id);
                take[i] = 1;
            }
            spans.push_back(std::move(span));
            owner.push_back(i);
        }
        if (spans.empty()) return;
        GenerationBatchResult r = runner->generationForwardSpans(spans);
        ++out.model_forward_batches;
        for (std::size_t k = 0; k < spans.size(); ++k) {
            auto const n = static_cast<std::uint32_t>(spans[k].token_ids.size());
            out.model_forward_tokens += n;
            (live[owner[k]]->record->prefilling() ? out.prefill_tokens : out.decode_tokens) += n;
        }
        if (!r.success || r.steps.size() != spans.size()) {
            std::string const text = r.detail.empty() ? "model returned an invalid span result" : r.detail;
            for (std::size_t k = 0; k < spans.size(); ++k) {
                finish(*live[owner[k]]->record, GenerationTerminalReason::Failed, GenerationError::ModelFailed, text);
            }
            return;
        }
        for (std::size_t k = 0; k < spans.size(); ++k) {
            Record& rec = *live[owner[k]]->record;
            bool const prefill = rec.prefilling();
            advance(rec, std::move(r.steps[k]), static_cast<std::uint32_t>(spans[k].token_ids.size()), prefill);
        }
    }

    EngineKvBackend* kv;
    GenerationModelRunner* runner;
    IterationSchedulerConfig config;
    std::atomic<bool> stopped{false};
    std::unordered_map<RequestId, Record> records;
    std::unordered_map<RequestId, SchedulerRequestState> states;
    std::deque<RequestId> queue;
    std::vector<GenerationTerminal> terminals;
    std::uint64_t iterations{0};
    std::uint64_t reserved_kv_tokens{0};
    std::uint64_t forward_tokens{0};
    std::uint64_t forward_batches{0};
    std::uint64_t prefill_tokens{0};
    std::uint64_t decode_tokens{0};
};

IterationSchedulerRuntime::IterationSchedulerRuntime(EngineKvBackend& kv_backend, GenerationModelRunner& model_runner,
                                                     IterationSchedulerConfig config)
    : impl_(std::make_unique<Impl>(kv_backend, model_runner, config))
{
}

IterationSchedulerRuntime::~IterationSchedulerRuntime()
{
    if (impl_ != nullptr) {
        impl_->stopped.store(true, std::memory_order_release);
        impl_->stopAll();
    }
}

SchedulerAdmissionResult IterationSchedulerRuntime::submit(GenerationRequest request)
{
    Impl& s = *impl_;
    RequestId const id = request.request_id;
    if (stopped()) return s.reject(id, SchedulerAdmissionError::RuntimeStopped, "runtime is stopped", true);
    if (s.states.count(id) != 0) {
        return s.reject(id, SchedulerAdmissionError::DuplicateRequest, "request id was already submitted", false);
    }
    if (!s.config.valid()) {
        return s.reject(id, SchedulerAdmissionError::InvalidArgument, "invalid scheduler configuration", true);
    }
    if (std::optional<std::string> bad = detail::validateRequest(s.runner->generationConfig(), request)) {
        return s.reject(id, SchedulerAdmissionError::InvalidArgument, std::move(*bad), true);
    }
    if (snapshot().activeCount() >= s.config.max_active_requests) {
        return s.reject(id, SchedulerAdmissionError::MaxActiveRequests, "max_active_requests reached", true);
    }
    // Worst case committed tokens: the prompt plus every completion token but the last.
    std::uint64_t const budget = request.prompt_token_ids.size() + request.sampling.max_new_tokens - 1ull;
    if (budget > s.config.max_kv_tokens || s.reserved_kv_tokens > s.config.max_kv_tokens - budget) {
        return s.reject(id, SchedulerAdmissionError::KvTokenBudget, "KV token budget exhausted", true);
    }
    try {
        Impl::Record record;
        record.request = std::move(request);
        record.state = SchedulerRequestState::Waiting;
        record.terminal.request_id = id;
        record.terminal.usage.prompt_tokens = static_cast<std::uint32_t>(record.request.prompt_token_ids.size());
        record.kv_budget = budget;
        record.progress.started = detail::Clock::now();
        s.records.emplace(id, std::move(record));
        try {
            s.states.emplace(id, SchedulerRequestState::Waiting);
            s.queue.push_back(id);
        } catch (...) {
            s.states.erase(id);
            s.records.erase(id);
            throw;
        }
    } catch (std::bad_alloc const&) {
        return {false, SchedulerAdmissionError::InternalError, "admission allocation failed"};
    }
    s.reserved_kv_tokens += budget;
    return {true, SchedulerAdmissionError::None, {}};
}

bool IterationSchedulerRuntime::cancel(RequestId request_id) noexcept
{
    auto it = impl_->records.find(request_id);
    if (it == impl_->records.end() || it->second.terminal_state()) return false;
    it->second.cancel_requested = true;
    impl_->setState(request_id, &it->second, SchedulerRequestState::Cancelling);
    return true;
}

SchedulerIterationResult IterationSchedulerRuntime::runIteration()
{
    Impl& s = *impl_;
    SchedulerIterationResult result;
    result.iteration = ++s.iterations;
    std::size_t const before = s.terminals.size();
    if (stopped()) {
        s.stopAll();
        result.terminals_produced = static_cast<std::uint32_t>(s.terminals.size() - before);
        return result;
    }

    std::vector<Impl::Selected> selected;
    std::size_t const take = std::min<std::size_t>(s.queue.size(), s.config.max_batched_tokens);
    try {
        selected.reserve(take);
        for (std::size_t i = 0; i < take; ++i) {
            RequestId const id = s.queue.front();
            s.queue.pop_front();
            auto it = s.records.find(id);
            if (it == s.records.end() || it->second.terminal_state()) continue;
            Impl::Record& r = it->second;
            auto const left = static_cast<std::uint32_t>(r.request.prompt_token_ids.size()) - r.prompt_position;
            selected.push_back({&r, left == 0 ? 1u : std::min(left, s.config.prefill_chunk_size)});
        }
    } catch (std::bad_alloc const&) {
        s.failAll(selected, GenerationError::InternalError, "iteration planning allocation failed");
    }

    std::uint32_t const max_batch = s.runner->generationMaxBatchSize();
    if (max_batch == 0) {
        s.failAll(selected, GenerationError::ModelFailed, "model runner reports a maximum batch size of zero");
    } else {
        try {
            if (s.runner->generationSupportsSpans()) {
                s.spanIteration(selected, s.config.max_batched_tokens, max_batch, result);
            } else {
                s.waveIteration(selected, s.config.max_batched_tokens, max_batch, result);
            }
        } catch (std::bad_alloc const&) {
            s.failAll(selected, GenerationError::InternalError, "model batch allocation failed");
        }
    }
    s.forward_tokens += result.model_forward_tokens;
    s.forward_batches += result.model_forward_batches;
    s.prefill_tokens += result.prefill_tokens;
    s.decode_tokens += result.decode_tokens;

    for (Impl::Selected const& sel : selected) {
        if (sel.record->terminal_state()) continue;
        if (stopped()) {
            s.stopRecord(*sel.record);
        } else {
            s.queue.push_back(sel.record->request.request_id);
        }
    }
    if (stopped()) s.stopAll();
    result.terminals_produced = static_cast<std::uint32_t>(s.terminals.size() - before);
    return result;
}

std::vector<GenerationTerminal> IterationSchedulerRuntime::drain()
{
    while (!idle()) {
        SchedulerIterationResult const r = runIteration();
        if (r.model_forward_tokens == 0 && r.terminals_produced == 0 && !stopped()) break;
    }
    return takeTerminals();
}

std::vector<GenerationTerminal> IterationSchedulerRuntime::takeTerminals()
{
    std::vector<GenerationTerminal> out;
    out.swap(impl_->terminals);
    return out;
}

std::optional<SchedulerRequestState> IterationSchedulerRuntime::requestState(RequestId request_id) const
{
    auto it = impl_->states.find(request_id);
    if (it == impl_->states.end()) return std::nullopt;
    return it->second;
}

IterationSchedulerSnapshot IterationSchedulerRuntime::snapshot() const
{
    Impl const& s = *impl_;
    IterationSchedulerSnapshot out;
    out.iteration_count = s.iterations;
    out.accepted_count = s.records.size();
    out.reserved_kv_tokens = s.reserved_kv_tokens;
    out.model_forward_tokens = s.forward_tokens;
    out.model_forward_batches = s.forward_batches;
    out.prefill_tokens = s.prefill_tokens;
    out.decode_tokens = s.decode_tokens;
    out.stopped = stopped();
    for (auto const& kv : s.states) {
        switch (kv.second) {
        case SchedulerRequestState::Created: break;
        case SchedulerRequestState::Waiting: ++out.waiting_count; break;
        case SchedulerRequestState::Running: ++out.running_count; break;
        case SchedulerRequestState::Cancelling: ++out.cancelling_count; break;
        case SchedulerRequestState::Terminal: ++out.terminal_count; break;
        case SchedulerRequestState::Rejected: ++out.rejected_count; break;
        }
    }
    return out;
}

bool IterationSchedulerRuntime::idle() const noexcept { return impl_->queue.empty(); }
void IterationSchedulerRuntime::stop() noexcept { impl_->stopped.store(true, std::memory_order_release); }
bool IterationSchedulerRuntime::stopped() const noexcept { return impl_->stopped.load(std::memory_order_acquire); }

}  // namespace kimkvcache
