// Generation SPI defaults and the single-request runtime
// (src/engine/generation.cpp:1-343 of the reference).
#include "kim-kv/engine/generation.h"

#include "generation_internal.h"

#include <algorithm>
#include <limits>
#include <new>
#include <utility>

namespace kimkvcache {

namespace detail {

std::optional<std::string> validateRequest(TinyLlamaConfig const& model, GenerationRequest const& request)
{
    if (!model.valid() || request.request_id == kInvalidRequestId || request.prompt_token_ids.empty()
        || request.sampling.max_new_tokens == 0) {
        return std::string("a valid model config, request id, non-empty prompt and max_new_tokens > 0 are required");
    }
    std::size_t const prompt = request.prompt_token_ids.size();
    if (prompt > model.max_position_embeddings
        || request.sampling.max_new_tokens > model.max_position_embeddings - prompt + 1) {
        return std::string("prompt plus completion exceed max_position_embeddings");
    }
    if (request.sampling.eos_token_id.value_or(model.eos_token_id) >= model.vocabulary_size) {
        return std::string("EOS token id is not in the vocabulary");
    }
    for (std::uint32_t token : request.prompt_token_ids) {
        if (token >= model.vocabulary_size) return std::string("prompt token id is not in the vocabulary");
    }
    return std::nullopt;
}

void completeTerminal(GenerationTerminal& terminal, RequestProgress& progress, EngineKvBackend& kv,
                      RequestId request_id, GenerationTerminalReason reason, GenerationError error,
                      std::string detail)
{
    terminal.reason = reason;
    terminal.error = error;
    terminal.detail = std::move(detail);
    terminal.usage.completion_tokens = static_cast<std::uint32_t>(terminal.output_token_ids.size());
    terminal.usage.total_tokens = terminal.usage.prompt_tokens + terminal.usage.completion_tokens;
    if (progress.kv_created) {
        progress.kv_created = false;
        EngineKvStatus const released = kv.releaseRequest(request_id);
        if (!released.ok()) {
            terminal.reason = GenerationTerminalReason::Failed;
            terminal.error = GenerationError::KvBackendFailed;
            terminal.detail = "KV request release failed: " + std::string(toString(released.error));
        }
    }
    terminal.metrics.e2e_ns = elapsedNs(progress.started, Clock::now());
    if (progress.emitted) {
        terminal.metrics.ttft_ns = elapsedNs(progress.started, progress.first_token);
        std::size_t const n = terminal.output_token_ids.size();
        if (n > 1) terminal.metrics.tpot_ns = elapsedNs(progress.first_token, progress.last_token) / (n - 1);
    }
}

}  // namespace detail

// ---- model SPI defaults --------------------------------------------------------

GenerationBatchResult GenerationModelRunner::generationForwardBatch(std::vector<GenerationBatchItem> const& batch)
{
    GenerationBatchResult result;
    if (batch.empty()) {
        result.detail = "empty generation batch";
        return result;
    }
    try {
        result.steps.reserve(batch.size());
        for (GenerationBatchItem const& item : batch) {
            result.steps.push_back(generationForwardToken(item.request_id, item.token_id, item.expected_position));
        }
    } catch (std::bad_alloc const&) {
        result.steps.clear();
        result.detail = "generation batch allocation failed";
        return result;
    }
    result.success = true;
    return result;
}

std::uint32_t GenerationModelRunner::generationMaxBatchSize() const noexcept
{
    return std::numeric_limits<std::uint32_t>::max();
}

bool GenerationModelRunner::generationSupportsSpans() const noexcept { return false; }

GenerationBatchResult GenerationModelRunner::generationForwardSpans(std::vector<GenerationSpan> const& spans)
{
    GenerationBatchResult result;
    if (spans.empty()) {
        result.detail = "empty generation span list";
        return result;
    }
    try {
        result.steps.assign(spans.size(), GenerationStepResult{});
        std::vector<bool> live(spans.size(), true);
        std::size_t longest = 0;
        for (GenerationSpan const& s : spans) {
            if (s.token_ids.empty()) {
                result.steps.clear();
                result.detail = "generation span without tokens";
                return result;
            }
            longest = std::max(longest, s.token_ids.size());
        }
        std::uint32_t const cap = std::max<std::uint32_t>(1, generationMaxBatchSize());
        std::vector<GenerationBatchItem> wave;
        std::vector<std::size_t> owner;
        for (std::size_t k = 0; k < longest; ++k) {
            wave.clear();
            owner.clear();
            for (std::size_t i = 0; i < spans.size(); ++i) {
                if (!live[i] || k >= spans[i].token_ids.size()) continue;
                wave.push_back(GenerationBatchItem{spans[i].request_id, spans[i].token_ids[k],
                                                   spans[i].first_position + static_cast<std::uint32_t>(k)});
                owner.push_back(i);
            }
            for (std::size_t b = 0; b < wave.size(); b += cap) {
                std::size_t const e = std::min(wave.size(), b + cap);
                std::vector<GenerationBatchItem> part(wave.begin() + static_cast<std::ptrdiff_t>(b),
                                                      wave.begin() + static_cast<std::ptrdiff_t>(e));
                GenerationBatchResult r = generationForwardBatch(part);
                bool const whole = r.success && r.steps.size() == part.size();
                for (std::size_t j = b; j < e; ++j) {
                    std::size_t const i = owner[j];
                    GenerationStepResult step = whole ? std::move(r.steps[j - b])
                                                      : GenerationStepResult{false, 0, r.detail.empty()
                                                                                 ? "model batch failed" : r.detail};
                    if (!step.success) live[i] = false;
                    result.steps[i] = std::move(step);
                }
            }
        }
    } catch (std::bad_alloc const&) {
        result.steps.clear();
        result.detail = "generation span allocation failed";
        return result;
    }
    result.success = true;
    return result;
}

void GenerationCancellationToken::cancel() noexcept { cancelled_.store(true, std::memory_order_release); }
bool GenerationCancellationToken::cancelled() const noexcept { return cancelled_.load(std::memory_order_acquire); }

// ---- single-request runtime ----------------------------------------------------

SingleRequestGenerationRuntime::SingleRequestGenerationRuntime(EngineKvBackend& kv_backend,
                                                               GenerationModelRunner& model_runner) noexcept
    : kv_backend_(&kv_backend), model_runner_(&model_runner)
{
}

void SingleRequestGenerationRuntime::stop() noexcept { stopped_.store(true, std::memory_order_release); }
bool SingleRequestGenerationRuntime::stopped() const noexcept { return stopped_.load(std::memory_order_acquire); }

GenerationTerminal SingleRequestGenerationRuntime::generate(GenerationRequest const& request)
{
    detail::RequestProgress progress;
    progress.started = detail::Clock::now();
    GenerationTerminal terminal;
    terminal.request_id = request.request_id;
    auto done = [&](GenerationTerminalReason reason, GenerationError error, std::string text) {
        detail::completeTerminal(terminal, progress, *kv_backend_, request.request_id, reason, error,
                                 std::move(text));
        return terminal;
    };

    bool idle = false;
    if (!generating_.compare_exchange_strong(idle, true, std::memory_order_acq_rel)) {
        return done(GenerationTerminalReason::Failed, GenerationError::InvalidArgument,
                    "the single-request runtime is already generating");
    }
    struct Release {
        std::atomic<bool>& flag;
        ~Release() { flag.store(false, std::memory_order_release); }
    } release{generating_};

    if (stopped()) return done(GenerationTerminalReason::RuntimeStopped, GenerationError::RuntimeStopped,
                               "runtime is stopped");
    TinyLlamaConfig const model = model_runner_->generationConfig();
    if (std::optional<std::string> bad = detail::validateRequest(model, request)) {
        if (!request.prompt_token_ids.empty() && request.sampling.max_new_tokens != 0 && model.valid()
            && request.request_id != kInvalidRequestId) {
            terminal.usage.prompt_tokens = static_cast<std::uint32_t>(request.prompt_token_ids.size());
        }
        return done(GenerationTerminalReason::Failed, GenerationError::InvalidArgument, std::move(*bad));
    }
    terminal.usage.prompt_tokens = static_cast<std::uint32_t>(request.prompt_token_ids.size());
    std::uint32_t const eos = request.sampling.eos_token_id.value_or(model.eos_token_id);
    auto cancelled = [&request] { return request.cancellation != nullptr && request.cancellation->cancelled(); };
    if (cancelled()) return done(GenerationTerminalReason::Cancelled, GenerationError::None,
                                 "cancelled before prefill");

    EngineKvStatus const created = kv_backend_->createRequest(request.request_id);
    if (!created.ok()) {
        return done(GenerationTerminalReason::Failed, GenerationError::KvBackendFailed,
                    "KV request creation failed: " + std::string(toString(created.error)));
    }
    progress.kv_created = true;

    // One forward step: position `position` holds `token`; returns false (after
    // completing the terminal) when the step failed.
    std::uint32_t next = 0;
    auto forward = [&](std::uint32_t token, std::uint32_t position) {
        GenerationStepResult step = model_runner_->generationForwardToken(request.request_id, token, position);
        if (!step.success) {
            done(GenerationTerminalReason::Failed, GenerationError::ModelFailed, std::move(step.detail));
            return false;
        }
        if (step.greedy_token_id >= model.vocabulary_size) {
            done(GenerationTerminalReason::Failed, GenerationError::ModelFailed,
                 "model returned a token id outside the vocabulary");
            return false;
        }
        next = step.greedy_token_id;
        return true;
    };

    std::uint32_t const prompt = terminal.usage.prompt_tokens;
    for (std::uint32_t position = 0; position < prompt; ++position) {
        if (stopped()) return done(GenerationTerminalReason::RuntimeStopped, GenerationError::RuntimeStopped,
                                   "runtime stopped during prefill");
        if (cancelled()) return done(GenerationTerminalReason::Cancelled, GenerationError::None,
                                     "cancelled during prefill");
        if (!forward(request.prompt_token_ids[position], position)) return terminal;
    }
    for (std::uint32_t generated = 0;; ++generated) {
        if (stopped()) return done(GenerationTerminalReason::RuntimeStopped, GenerationError::RuntimeStopped,
                                   "runtime stopped during decode");
        if (cancelled()) return done(GenerationTerminalReason::Cancelled, GenerationError::None,
                                     "cancelled during decode");
        try {
            terminal.output_token_ids.push_back(next);
        } catch (std::bad_alloc const&) {
            return done(GenerationTerminalReason::Failed, GenerationError::InternalError,
                        "completion token allocation failed");
        }
        progress.tokenEmitted();
        if (next == eos) return done(GenerationTerminalReason::EosToken, GenerationError::None, "EOS token generated");
        if (generated + 1 == request.sampling.max_new_tokens) {
            return done(GenerationTerminalReason::MaxNewTokens, GenerationError::None, "max_new_tokens reached");
        }
        if (!forward(next, prompt + generated)) return terminal;
    }
}

}  // namespace kimkvcache
