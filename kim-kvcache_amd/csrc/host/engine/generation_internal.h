// Shared pieces of the single-request runtime and the iteration scheduler:
// request validation and terminal completion (usage, release of the KV
// request, TTFT / TPOT / end-to-end metrics).
#pragma once

#include "kim-kv/engine/generation.h"

#include <chrono>
#include <optional>
#include <string>

namespace kimkvcache::detail {

using Clock = std::chrono::steady_clock;

inline std::uint64_t elapsedNs(Clock::time_point begin, Clock::time_point end) noexcept
{
    auto const ns = std::chrono::duration_cast<std::chrono::nanoseconds>(end - begin).count();
    return ns > 0 ? static_cast<std::uint64_t>(ns) : 0;
}

// The request-shape checks of src/engine/generation.cpp:160-205 and
// src/engine/iteration_scheduler.cpp:83-118, in their order; nullopt = valid.
std::optional<std::string> validateRequest(TinyLlamaConfig const& model, GenerationRequest const& request);

// Per-request progress shared by both runtimes.
struct RequestProgress {
    Clock::time_point started{};
    Clock::time_point first_token{};
    Clock::time_point last_token{};
    bool emitted{false};
    bool kv_created{false};

    void tokenEmitted() noexcept
    {
        last_token = Clock::now();
        if (!emitted) {
            first_token = last_token;
            emitted = true;
        }
    }
};

// Fills reason / error / detail / usage / metrics and releases the KV request
// when one was created (a failed release turns the terminal into a
// KvBackendFailed failure).
void completeTerminal(GenerationTerminal& terminal, RequestProgress& progress, EngineKvBackend& kv,
                      RequestId request_id, GenerationTerminalReason reason, GenerationError error,
                      std::string detail);

}  // namespace kimkvcache::detail
