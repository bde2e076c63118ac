#pragma once

// Iteration-level FIFO scheduler over the engine SPI and the generation SPI
// (include/kim-kv/engine/iteration_scheduler.h:1-183 of the reference: same
// names, enums, config and result fields).  With a runner that supports
// spans, each iteration's prompt chunks and decode steps go to the runner as
// one mixed call (chunked prefill in one launch per layer); otherwise the
// iteration runs the reference's position waves.

#include "kim-kv/engine/generation.h"

#include <atomic>
#include <cstdint>
#include <memory>
#include <optional>
#include <string>
#include <string_view>
#include <vector>

namespace kimkvcache {

enum class SchedulerRequestState : std::uint8_t {
    Created,
    Waiting,
    Running,
    Cancelling,
    Terminal,
    Rejected,
};

[[nodiscard]] constexpr std::string_view toString(SchedulerRequestState state) noexcept
{
    switch (state) {
    case SchedulerRequestState::Created: return "created";
    case SchedulerRequestState::Waiting: return "waiting";
    case SchedulerRequestState::Running: return "running";
    case SchedulerRequestState::Cancelling: return "cancelling";
    case SchedulerRequestState::Terminal: return "terminal";
    case SchedulerRequestState::Rejected: return "rejected";
    }
    return "unknown";
}

enum class SchedulerAdmissionError : std::uint8_t {
    None,
    InvalidArgument,
    RuntimeStopped,
    DuplicateRequest,
    MaxActiveRequests,
    KvTokenBudget,
    InternalError,
};

[[nodiscard]] constexpr std::string_view toString(SchedulerAdmissionError error) noexcept
{
    switch (error) {
    case SchedulerAdmissionError::None: return "none";
    case SchedulerAdmissionError::InvalidArgument: return "invalid_argument";
    case SchedulerAdmissionError::RuntimeStopped: return "runtime_stopped";
    case SchedulerAdmissionError::DuplicateRequest: return "duplicate_request";
    case SchedulerAdmissionError::MaxActiveRequests: return "max_active_requests";
    case SchedulerAdmissionError::KvTokenBudget: return "kv_token_budget";
    case SchedulerAdmissionError::InternalError: return "internal_error";
    }
    return "unknown";
}

struct IterationSchedulerConfig final {
    std::uint32_t max_active_requests{0};
    // Sequence positions of all model calls of one iteration.
    std::uint32_t max_batched_tokens{0};
    // Worst-case committed tokens (prompt + max_new_tokens - 1) reserved at admission.
    std::uint64_t max_kv_tokens{0};
    // Prompt positions a prefilling request may advance in one iteration
    // (decode requests advance by one).
    std::uint32_t prefill_chunk_size{16};

    [[nodiscard]] constexpr bool valid() const noexcept
    {
        return max_active_requests != 0 && max_batched_tokens != 0 && max_kv_tokens != 0 && prefill_chunk_size != 0;
    }
};

struct SchedulerAdmissionResult final {
    bool accepted{false};
    SchedulerAdmissionError error{SchedulerAdmissionError::InternalError};
    std::string detail{};

    [[nodiscard]] bool ok() const noexcept { return accepted && error == SchedulerAdmissionError::None; }
};

struct SchedulerIterationResult final {
    std::uint64_t iteration{0};
    std::uint32_t model_forward_tokens{0};
    std::uint32_t model_forward_batches{0};
    std::uint32_t prefill_tokens{0};
    std::uint32_t decode_tokens{0};
    std::uint32_t terminals_produced{0};
};

struct IterationSchedulerSnapshot final {
    std::uint64_t iteration_count{0};
    std::uint64_t accepted_count{0};
    std::uint64_t rejected_count{0};
    std::uint64_t waiting_count{0};
    std::uint64_t running_count{0};
    std::uint64_t cancelling_count{0};
    std::uint64_t terminal_count{0};
    std::uint64_t reserved_kv_tokens{0};
    std::uint64_t model_forward_tokens{0};
    std::uint64_t model_forward_batches{0};
    std::uint64_t prefill_tokens{0};
    std::uint64_t decode_tokens{0};
    bool stopped{false};

    [[nodiscard]] constexpr std::uint64_t activeCount() const noexcept
    {
        return waiting_count + running_count + cancelling_count;
    }
};

// submit / cancel / runIteration / drain are externally serialised; stop() is
// thread-safe and observed at the current token boundary; drain() then
// produces every remaining terminal.
class IterationSchedulerRuntime final {
public:
    IterationSchedulerRuntime(EngineKvBackend& kv_backend, GenerationModelRunner& model_runner,
                              IterationSchedulerConfig config);
    ~IterationSchedulerRuntime();

    IterationSchedulerRuntime(IterationSchedulerRuntime const&) = delete;
    IterationSchedulerRuntime& operator=(IterationSchedulerRuntime const&) = delete;

    [[nodiscard]] SchedulerAdmissionResult submit(GenerationRequest request);
    [[nodiscard]] bool cancel(RequestId request_id) noexcept;
    [[nodiscard]] SchedulerIterationResult runIteration();

    // Runs until every accepted request has its one terminal; includes
    // terminals completed before the call.
    [[nodiscard]] std::vector<GenerationTerminal> drain();

    // Destructive: a terminal is delivered once.
    [[nodiscard]] std::vector<GenerationTerminal> takeTerminals();

    [[nodiscard]] std::optional<SchedulerRequestState> requestState(RequestId request_id) const;
    [[nodiscard]] IterationSchedulerSnapshot snapshot() const;
    [[nodiscard]] bool idle() const noexcept;

    void stop() noexcept;
    [[nodiscard]] bool stopped() const noexcept;

private:
    class Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace kimkvcache
