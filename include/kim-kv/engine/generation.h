#pragma once

// Generation SPI and the single-request runtime
// (include/kim-kv/engine/generation.h:1-204 of the reference: same names,
// enums, fields and contracts), plus one addition: spans, so a runner that
// can attend a whole prompt chunk in one launch (the MFMA chunked-prefill
// path) receives it as one item instead of one item per position.

#include "kim-kv/engine/engine_kv.h"
#include "kim-kv/model/tinyllama_config.h"

#include <atomic>
#include <cstdint>
#include <memory>
#include <optional>
#include <string>
#include <string_view>
#include <vector>

namespace kimkvcache {

enum class GenerationError : std::uint8_t {
    None,
    InvalidArgument,
    RuntimeStopped,
    ModelFailed,
    KvBackendFailed,
    InternalError,
};

[[nodiscard]] constexpr std::string_view toString(GenerationError error) noexcept
{
    switch (error) {
    case GenerationError::None: return "none";
    case GenerationError::InvalidArgument: return "invalid_argument";
    case GenerationError::RuntimeStopped: return "runtime_stopped";
    case GenerationError::ModelFailed: return "model_failed";
    case GenerationError::KvBackendFailed: return "kv_backend_failed";
    case GenerationError::InternalError: return "internal_error";
    }
    return "unknown";
}

enum class GenerationTerminalReason : std::uint8_t {
    EosToken,
    MaxNewTokens,
    Cancelled,
    RuntimeStopped,
    Failed,
};

[[nodiscard]] constexpr std::string_view toString(GenerationTerminalReason reason) noexcept
{
    switch (reason) {
    case GenerationTerminalReason::EosToken: return "eos_token";
    case GenerationTerminalReason::MaxNewTokens: return "max_new_tokens";
    case GenerationTerminalReason::Cancelled: return "cancelled";
    case GenerationTerminalReason::RuntimeStopped: return "runtime_stopped";
    case GenerationTerminalReason::Failed: return "failed";
    }
    return "unknown";
}

// Greedy decoding; eos_token_id unset = the model's EOS token.
struct SamplingConfig final {
    std::uint32_t max_new_tokens{0};
    std::optional<std::uint32_t> eos_token_id{};
};

class GenerationCancellationToken final {
public:
    void cancel() noexcept;
    [[nodiscard]] bool cancelled() const noexcept;

private:
    std::atomic<bool> cancelled_{false};
};

struct GenerationRequest final {
    RequestId request_id{kInvalidRequestId};
    std::vector<std::uint32_t> prompt_token_ids{};
    SamplingConfig sampling{};
    std::shared_ptr<GenerationCancellationToken> cancellation{};
};

struct GenerationUsage final {
    std::uint32_t prompt_tokens{0};
    std::uint32_t completion_tokens{0};
    std::uint32_t total_tokens{0};
};

struct GenerationMetrics final {
    std::uint64_t ttft_ns{0};
    std::uint64_t tpot_ns{0};
    std::uint64_t e2e_ns{0};
};

struct GenerationTerminal final {
    RequestId request_id{kInvalidRequestId};
    GenerationTerminalReason reason{GenerationTerminalReason::Failed};
    GenerationError error{GenerationError::InternalError};
    std::string detail{};
    std::vector<std::uint32_t> output_token_ids{};
    GenerationUsage usage{};
    GenerationMetrics metrics{};

    [[nodiscard]] bool ok() const noexcept
    {
        return error == GenerationError::None
            && (reason == GenerationTerminalReason::EosToken || reason == GenerationTerminalReason::MaxNewTokens);
    }
};

struct GenerationStepResult final {
    bool success{false};
    std::uint32_t greedy_token_id{0};
    std::string detail{};
};

struct GenerationBatchItem final {
    RequestId request_id{kInvalidRequestId};
    std::uint32_t token_id{0};
    std::uint32_t expected_position{0};
};

struct GenerationBatchResult final {
    bool success{false};
    std::vector<GenerationStepResult> steps{};
    std::string detail{};
};

// Consecutive positions [first_position, first_position + token_ids.size())
// of one request in one model call (no reference counterpart).  A decode step
// is a span of one token; a prompt chunk a span of several.  The step result
// of a span is the greedy token after its last position.
struct GenerationSpan final {
    RequestId request_id{kInvalidRequestId};
    std::uint32_t first_position{0};
    std::vector<std::uint32_t> token_ids{};
};

// Narrow model SPI (generation.h:147-180 of the reference): the greedy next
// token only; logits stay runner-specific.
class GenerationModelRunner {
public:
    virtual ~GenerationModelRunner() = default;

    GenerationModelRunner(GenerationModelRunner const&) = delete;
    GenerationModelRunner& operator=(GenerationModelRunner const&) = delete;

    [[nodiscard]] virtual TinyLlamaConfig generationConfig() const noexcept = 0;
    [[nodiscard]] virtual GenerationStepResult generationForwardToken(RequestId request_id, std::uint32_t token_id,
                                                                      std::uint32_t expected_position) = 0;

    // Independent positions as one model batch.  The default forwards each
    // item through generationForwardToken().  A successful result has exactly
    // batch.size() steps; request-local failures are failed steps.
    [[nodiscard]] virtual GenerationBatchResult generationForwardBatch(std::vector<GenerationBatchItem> const& batch);

    [[nodiscard]] virtual std::uint32_t generationMaxBatchSize() const noexcept;

    // Spans (addition).  A runner that returns true from
    // generationSupportsSpans() receives whole prompt chunks from the
    // iteration scheduler; generationMaxBatchSize() then bounds the positions
    // of one call.  The default generationForwardSpans() runs the spans as
    // position waves through generationForwardBatch() (wave k holds position
    // k of every span longer than k; a span that fails leaves later waves).
    [[nodiscard]] virtual bool generationSupportsSpans() const noexcept;
    [[nodiscard]] virtual GenerationBatchResult generationForwardSpans(std::vector<GenerationSpan> const& spans);

protected:
    GenerationModelRunner() = default;
    GenerationModelRunner(GenerationModelRunner&&) noexcept = default;
    GenerationModelRunner& operator=(GenerationModelRunner&&) noexcept = default;
};

// One synchronous request at a time (generation.h:182-202 of the reference);
// stop() is thread-safe and observed at token boundaries.
class SingleRequestGenerationRuntime final {
public:
    SingleRequestGenerationRuntime(EngineKvBackend& kv_backend, GenerationModelRunner& model_runner) noexcept;

    SingleRequestGenerationRuntime(SingleRequestGenerationRuntime const&) = delete;
    SingleRequestGenerationRuntime& operator=(SingleRequestGenerationRuntime const&) = delete;

    [[nodiscard]] GenerationTerminal generate(GenerationRequest const& request);

    void stop() noexcept;
    [[nodiscard]] bool stopped() const noexcept;

private:
    EngineKvBackend* kv_backend_{nullptr};
    GenerationModelRunner* model_runner_{nullptr};
    std::atomic<bool> stopped_{false};
    std::atomic<bool> generating_{false};
};

}  // namespace kimkvcache
