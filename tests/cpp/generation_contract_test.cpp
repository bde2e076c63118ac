// Contract tests of the single-request generation runtime and the iteration
// scheduler against a fake KV backend and a fake model (the scenarios of the
// reference's tests/engine/generation_runtime_test.cpp and
// tests/engine/iteration_scheduler_test.cpp), plus the span path: a runner
// that takes whole prompt chunks must produce the same tokens, terminals and
// budgets, with one model call per iteration.
//
// Built by kim-kvcache_amd/build.py against libkimkv.so; run by
// tests/test_cpp_contracts.py.  Prints one line per failed expectation.
#include "kim-kv/engine/iteration_scheduler.h"

#include <algorithm>
#include <cstdint>
#include <iostream>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

using namespace kimkvcache;

namespace {

int g_failures = 0;

void check(bool ok, std::string const& what)
{
    if (!ok) {
        std::cerr << "FAIL: " << what << '\n';
        ++g_failures;
    }
}

class FakeBackend final : public EngineKvBackend {
public:
    std::set<RequestId> refuse_create;

    EngineKvBackendKind kind() const noexcept override { return EngineKvBackendKind::Heterogeneous; }
    EngineKvConfig config() const noexcept override { return {}; }
    EngineKvStatus createRequest(RequestId id) override
    {
        if (id == kInvalidRequestId) return {EngineKvError::InvalidArgument};
        if (refuse_create.count(id)) return {EngineKvError::ResourceExhausted};
        return live_.insert(id).second ? EngineKvStatus{} : EngineKvStatus{EngineKvError::RequestAlreadyExists};
    }
    EngineKvStatus forkRequest(RequestId, RequestId) override { return {EngineKvError::InvalidState}; }
    EngineKvStatus releaseRequest(RequestId id) override
    {
        return live_.erase(id) ? EngineKvStatus{} : EngineKvStatus{EngineKvError::RequestNotFound};
    }
    TokenReserveResult reserveToken(ReserveTokenRequest const&) override
    {
        TokenReserveResult r;
        r.status = {EngineKvError::InvalidState};
        return r;
    }
    EngineKvBackendSnapshot snapshot() const override
    {
        EngineKvBackendSnapshot s;
        s.request_count = live_.size();
        return s;
    }
    bool checkInvariants() const override { return true; }

private:
    std::set<RequestId> live_;
};

// Greedy "model": next = (token * 7 + position * 3 + 1) % 251.
std::uint32_t rule(std::uint32_t token, std::uint32_t position) { return (token * 7 + position * 3 + 1) % 251; }

class FakeRunner final : public GenerationModelRunner {
public:
    TinyLlamaConfig model{8, 16, 2, 4, 2, 2, 256, 256, 1, 255, 1.0e-5F, 10000.0F, false};
    bool spans{false};
    std::uint32_t max_batch{0xFFFFFFFFu};
    std::set<RequestId> fail_requests;
    std::map<RequestId, std::uint64_t> positions;   // positions forwarded per request
    std::vector<std::size_t> batch_sizes;             // items per batch call (waves)
    std::vector<std::size_t> span_calls;              // positions per span call
    std::uint64_t calls{0};
    std::uint64_t fail_call{0}, force_call{0}, action_call{0};
    std::uint32_t forced{0};
    std::shared_ptr<GenerationCancellationToken> cancel_at_action;
    SingleRequestGenerationRuntime* stop_runtime{nullptr};
    IterationSchedulerRuntime* stop_scheduler{nullptr};
    RequestId stop_on{kInvalidRequestId};

    TinyLlamaConfig generationConfig() const noexcept override { return model; }
    std::uint32_t generationMaxBatchSize() const noexcept override { return max_batch; }
    bool generationSupportsSpans() const noexcept override { return spans; }

    GenerationStepResult generationForwardToken(RequestId id, std::uint32_t token, std::uint32_t position) override
    {
        ++calls;
        ++positions[id];
        if (action_call != 0 && calls == action_call) {
            if (cancel_at_action) cancel_at_action->cancel();
            if (stop_runtime) stop_runtime->stop();
        }
        if (stop_scheduler != nullptr && id == stop_on) stop_scheduler->stop();
        if (fail_call != 0 && calls == fail_call) return {false, 0, "injected model failure"};
        if (fail_requests.count(id)) return {false, 0, "injected request-local failure"};
        if (force_call != 0 && calls == force_call) return {true, forced, {}};
        return {true, rule(token, position), {}};
    }
    GenerationBatchResult generationForwardBatch(std::vector<GenerationBatchItem> const& batch) override
    {
        batch_sizes.push_back(batch.size());
        return GenerationModelRunner::generationForwardBatch(batch);
    }
    GenerationBatchResult generationForwardSpans(std::vector<GenerationSpan> const& s) override
    {
        std::size_t n = 0;
        for (GenerationSpan const& x : s) n += x.token_ids.size();
        span_calls.push_back(n);
        // A chunk-capable model computes every position of a span in one go;
        // the step is the token after the span's last position.
        GenerationBatchResult r;
        r.success = true;
        for (GenerationSpan const& x : s) {
            GenerationStepResult step{true, 0, {}};
            for (std::size_t k = 0; k < x.token_ids.size(); ++k) {
                step = generationForwardToken(x.request_id, x.token_ids[k],
                                              x.first_position + static_cast<std::uint32_t>(k));
                if (!step.success) break;
            }
            r.steps.push_back(step);
        }
        return r;
    }
};

std::vector<std::uint32_t> prompt(std::uint32_t n)
{
    std::vector<std::uint32_t> t(n);
    for (std::uint32_t i = 0; i < n; ++i) t[i] = (i * 11 + 3) % 251;
    return t;
}

std::vector<std::uint32_t> expectedTokens(std::vector<std::uint32_t> const& in, std::uint32_t out)
{
    std::uint32_t next = 0;
    for (std::uint32_t p = 0; p < in.size(); ++p) next = rule(in[p], p);
    std::vector<std::uint32_t> r;
    for (std::uint32_t g = 0; g < out; ++g) {
        r.push_back(next);
        next = rule(next, static_cast<std::uint32_t>(in.size()) + g);
    }
    return r;
}

GenerationRequest req(RequestId id, std::uint32_t in, std::uint32_t out)
{
    return GenerationRequest{id, prompt(in), SamplingConfig{out, 255}, {}};
}

std::map<RequestId, GenerationTerminal> byId(std::vector<GenerationTerminal> v)
{
    std::map<RequestId, GenerationTerminal> m;
    for (auto& t : v) m.emplace(t.request_id, std::move(t));
    return m;
}

void checkReclaimed(FakeBackend const& kv, IterationSchedulerRuntime const& s, std::string const& ctx)
{
    check(kv.snapshot().request_count == 0, ctx + ": KV requests released");
    IterationSchedulerSnapshot const snap = s.snapshot();
    check(snap.activeCount() == 0 && snap.reserved_kv_tokens == 0, ctx + ": scheduler budgets restored");
}

// ---- single-request runtime (generation_runtime_test.cpp) ----------------------------

void singleRequest()
{
    {
        FakeBackend kv;
        FakeRunner m;
        SingleRequestGenerationRuntime rt(kv, m);
        GenerationRequest a = req(1, 32, 1);
        GenerationTerminal t = rt.generate(a);
        check(t.ok() && t.reason == GenerationTerminalReason::MaxNewTokens, "ISL32/OSL1 ends on length");
        check(t.output_token_ids == expectedTokens(a.prompt_token_ids, 1), "ISL32/OSL1 tokens");
        check(t.usage.prompt_tokens == 32 && t.usage.completion_tokens == 1 && t.usage.total_tokens == 33,
              "ISL32/OSL1 usage");
        check(t.metrics.tpot_ns == 0, "one token has no TPOT");
        GenerationRequest b = req(2, 128, 32);
        t = rt.generate(b);
        check(t.ok() && t.output_token_ids == expectedTokens(b.prompt_token_ids, 32), "ISL128/OSL32 tokens");
        check(t.usage.total_tokens == 160 && t.metrics.e2e_ns >= t.metrics.ttft_ns, "ISL128/OSL32 usage and metrics");
        check(kv.snapshot().request_count == 0, "single runtime releases requests");
    }
    {
        FakeBackend kv;
        FakeRunner m;
        m.force_call = 4;
        m.forced = m.model.eos_token_id;
        SingleRequestGenerationRuntime rt(kv, m);
        GenerationRequest a = req(3, 4, 32);
        a.sampling.eos_token_id.reset();
        GenerationTerminal t = rt.generate(a);
        check(t.ok() && t.reason == GenerationTerminalReason::EosToken, "EOS terminal");
        check(t.output_token_ids == std::vector<std::uint32_t>{255} && t.usage.completion_tokens == 1,
              "EOS returned once and counted");
    }
    {
        FakeBackend kv;
        FakeRunner m;
        auto token = std::make_shared<GenerationCancellationToken>();
        m.cancel_at_action = token;
        m.action_call = 5;
        SingleRequestGenerationRuntime rt(kv, m);
        GenerationRequest a = req(4, 16, 8);
        a.cancellation = token;
        GenerationTerminal t = rt.generate(a);
        check(!t.ok() && t.reason == GenerationTerminalReason::Cancelled, "cancellation terminal");
        check(kv.snapshot().request_count == 0, "cancellation releases");
    }
    {
        FakeBackend kv;
        FakeRunner m;
        SingleRequestGenerationRuntime rt(kv, m);
        m.stop_runtime = &rt;
        m.action_call = 5;
        GenerationTerminal t = rt.generate(req(5, 16, 8));
        check(t.reason == GenerationTerminalReason::RuntimeStopped && t.error == GenerationError::RuntimeStopped,
              "stop terminal");
        check(rt.stopped() && rt.generate(req(6, 2, 1)).reason == GenerationTerminalReason::RuntimeStopped,
              "stopped runtime refuses work");
        check(kv.snapshot().request_count == 0, "stop releases");
    }
    {
        FakeBackend kv;
        FakeRunner m;
        m.fail_call = 3;
        SingleRequestGenerationRuntime rt(kv, m);
        GenerationTerminal t = rt.generate(req(7, 8, 2));
        check(t.error == GenerationError::ModelFailed && t.detail == "injected model failure",
              "model failure keeps its detail");
        m.fail_call = 0;
        GenerationRequest empty = req(8, 1, 1);
        empty.prompt_token_ids.clear();
        check(rt.generate(empty).error == GenerationError::InvalidArgument, "empty prompt refused");
        check(rt.generate(req(9, 256, 2)).error == GenerationError::InvalidArgument, "position overflow refused");
        GenerationRequest eos = req(10, 1, 1);
        eos.sampling.eos_token_id = 256;
        check(rt.generate(eos).error == GenerationError::InvalidArgument, "EOS outside vocabulary refused");
        m.force_call = m.calls + 1;
        m.forced = m.model.vocabulary_size;
        check(rt.generate(req(11, 1, 1)).error == GenerationError::ModelFailed, "model token outside vocabulary");
        check(kv.snapshot().request_count == 0, "failures release");
    }
    {
        FakeBackend kv;
        FakeRunner m;
        SingleRequestGenerationRuntime rt(kv, m);
        bool all = true;
        for (RequestId id = 100; id < 200; ++id) all = all && rt.generate(req(id, 32, 32)).ok();
        check(all && kv.snapshot().request_count == 0, "100 generations in a row");
    }
}

// ---- iteration scheduler (iteration_scheduler_test.cpp), both execution forms --------

void concurrency(bool spans)
{
    for (std::uint32_t c : {1u, 2u, 4u}) {
        FakeBackend kv;
        FakeRunner m;
        m.spans = spans;
        IterationSchedulerRuntime s(kv, m, {c, c, 4096});
        std::map<RequestId, GenerationRequest> sent;
        for (std::uint32_t i = 0; i < c; ++i) {
            GenerationRequest r = req(100 + i, 2 + i, 4 + i);
            sent.emplace(r.request_id, r);
            check(s.submit(std::move(r)).ok(), "concurrency: accepted");
        }
        auto done = byId(s.drain());
        check(done.size() == c, "concurrency: one terminal per request");
        for (auto const& e : sent) {
            auto it = done.find(e.first);
            check(it != done.end() && it->second.ok()
                      && it->second.output_token_ids
                          == expectedTokens(e.second.prompt_token_ids, e.second.sampling.max_new_tokens),
                  "concurrency: tokens match the greedy rule");
        }
        check(s.takeTerminals().empty(), "concurrency: terminals delivered once");
        if (spans) {
            check(!m.span_calls.empty() && m.span_calls.front() == c, "concurrency: first iteration is one call");
        } else {
            check(!m.batch_sizes.empty() && m.batch_sizes.front() == c, "concurrency: first wave is one batch");
        }
        checkReclaimed(kv, s, "concurrency");
    }
}

void dynamicJoin(bool spans)
{
    FakeBackend kv;
    FakeRunner m;
    m.spans = spans;
    IterationSchedulerRuntime s(kv, m, {4, 2, 4096});
    check(s.submit(req(1, 6, 2)).ok(), "join: long request");
    SchedulerIterationResult first = s.runIteration();
    check(first.model_forward_tokens == 2 && first.prefill_tokens == 2, "join: 2-token chunk under budget 2");
    check(s.submit(req(2, 1, 1)).ok() && s.submit(req(3, 2, 2)).ok(), "join: late requests");
    SchedulerIterationResult second = s.runIteration();
    check(second.model_forward_tokens <= 2, "join: budget respected");
    auto early = s.takeTerminals();
    check(early.size() == 1 && early.front().request_id == 2, "join: short request leaves first");
    check(s.requestState(1) == SchedulerRequestState::Running, "join: long request still running");
    check(s.drain().size() == 2, "join: the rest terminate once");
    checkReclaimed(kv, s, "join");
}

void chunkedPrefill(bool spans)
{
    FakeBackend kv;
    FakeRunner m;
    m.spans = spans;
    IterationSchedulerRuntime s(kv, m, {2, 6, 4096, 3});
    check(s.submit(req(40, 5, 2)).ok() && s.submit(req(41, 5, 2)).ok(), "chunked: accepted");
    SchedulerIterationResult first = s.runIteration();
    check(first.model_forward_tokens == 6 && first.prefill_tokens == 6 && first.decode_tokens == 0,
          "chunked: 3 prompt positions each");
    check(m.positions[40] == 3 && m.positions[41] == 3, "chunked: quota per request");
    if (spans) {
        check(first.model_forward_batches == 1 && m.span_calls == std::vector<std::size_t>{6},
              "chunked: one mixed call holds both chunks");
    } else {
        check(first.model_forward_batches == 3 && m.batch_sizes == std::vector<std::size_t>(3, 2),
              "chunked: three two-request waves");
    }
    auto done = s.drain();
    check(done.size() == 2 && std::all_of(done.begin(), done.end(), [](auto const& t) { return t.ok(); }),
          "chunked: both complete");
    for (auto const& t : done) {
        check(t.output_token_ids == expectedTokens(prompt(5), 2), "chunked: tokens match the greedy rule");
    }
    IterationSchedulerSnapshot snap = s.snapshot();
    check(snap.prefill_tokens == 10 && snap.decode_tokens == 2 && snap.model_forward_tokens == 12,
          "chunked: cumulative accounting");
    check(snap.model_forward_batches == (spans ? 3u : 6u), "chunked: cumulative calls");
    checkReclaimed(kv, s, "chunked");
}

void admission()
{
    FakeBackend kv;
    FakeRunner m;
    IterationSchedulerRuntime s(kv, m, {2, 1, 8});
    check(s.submit(req(10, 2, 2)).ok(), "admission: first");
    check(s.submit(req(10, 1, 1)).error == SchedulerAdmissionError::DuplicateRequest, "admission: duplicate");
    check(s.submit(req(11, 2, 2)).ok(), "admission: second");
    check(s.submit(req(12, 1, 1)).error == SchedulerAdmissionError::MaxActiveRequests, "admission: active gate");
    (void)s.drain();
    check(s.submit(req(13, 8, 2)).error == SchedulerAdmissionError::KvTokenBudget, "admission: KV budget gate");
    GenerationRequest bad = req(14, 1, 1);
    bad.prompt_token_ids.clear();
    check(s.submit(std::move(bad)).error == SchedulerAdmissionError::InvalidArgument, "admission: invalid");
    check(s.requestState(12) == SchedulerRequestState::Rejected && s.requestState(13) == SchedulerRequestState::Rejected,
          "admission: rejected state recorded");
    check(s.snapshot().accepted_count == 2, "admission: rejected never accepted");
    checkReclaimed(kv, s, "admission");
}

void isolation(bool spans)
{
    FakeBackend kv;
    FakeRunner m;
    m.spans = spans;
    m.fail_requests.insert(22);
    kv.refuse_create.insert(23);
    IterationSchedulerRuntime s(kv, m, {4, 4, 4096});
    for (RequestId id : {20u, 21u, 22u, 23u}) check(s.submit(req(id, 2, 2)).ok(), "isolation: accepted");
    check(s.cancel(21) && s.requestState(21) == SchedulerRequestState::Cancelling, "isolation: cancelling");
    auto done = byId(s.drain());
    check(done.size() == 4, "isolation: four terminals");
    check(done[20].ok(), "isolation: healthy request completes");
    check(done[21].reason == GenerationTerminalReason::Cancelled, "isolation: cancelled");
    check(done[22].error == GenerationError::ModelFailed, "isolation: model failure stays local");
    check(done[23].error == GenerationError::KvBackendFailed, "isolation: KV failure stays local");
    checkReclaimed(kv, s, "isolation");
}

void stopAndPressure(bool spans)
{
    {
        FakeBackend kv;
        FakeRunner m;
        m.spans = spans;
        IterationSchedulerRuntime s(kv, m, {4, 4, 4096});
        m.stop_scheduler = &s;
        m.stop_on = 30;
        check(s.submit(req(30, 4, 4)).ok() && s.submit(req(31, 4, 4)).ok(), "stop: accepted");
        auto done = s.drain();
        check(done.size() == 2 && std::all_of(done.begin(), done.end(), [](auto const& t) {
                  return t.reason == GenerationTerminalReason::RuntimeStopped;
              }),
              "stop: every active request stopped once");
        check(s.submit(req(32, 1, 1)).error == SchedulerAdmissionError::RuntimeStopped, "stop: refuses new work");
        checkReclaimed(kv, s, "stop");
    }
    FakeBackend kv;
    FakeRunner m;
    m.spans = spans;
    IterationSchedulerRuntime s(kv, m, {4, 4, 4096});
    bool ok = true;
    for (std::uint32_t w = 0; w < 25; ++w) {
        for (std::uint32_t i = 0; i < 4; ++i) ok = ok && s.submit(req(1000 + w * 4 + i, 2, 2)).ok();
        ok = ok && s.drain().size() == 4;
    }
    check(ok && s.snapshot().accepted_count == 100, "pressure: 25 waves of 4");
    checkReclaimed(kv, s, "pressure");
}

void destructorReclaims()
{
    FakeBackend kv;
    FakeRunner m;
    {
        IterationSchedulerRuntime s(kv, m, {2, 2, 64});
        check(s.submit(req(2000, 4, 4)).ok(), "destructor: accepted");
        (void)s.runIteration();
        check(kv.snapshot().request_count == 1, "destructor: request live");
    }
    check(kv.snapshot().request_count == 0, "destructor: request released");
}

// Span-only: a long prompt advances by whole chunks, mixed with decode lanes in the same call.
void mixedSpans()
{
    FakeBackend kv;
    FakeRunner m;
    m.spans = true;
    IterationSchedulerRuntime s(kv, m, {8, 64, 1 << 16, 16});
    check(s.submit(req(1, 3, 6)).ok(), "mixed: short request");
    (void)s.runIteration();   // request 1 finishes its prompt
    check(s.submit(req(2, 40, 3)).ok(), "mixed: long prompt joins");
    SchedulerIterationResult it = s.runIteration();
    check(it.model_forward_batches == 1 && it.decode_tokens == 1 && it.prefill_tokens == 16,
          "mixed: one call with a decode step and a 16-token chunk");
    auto done = byId(s.drain());
    check(done[1].ok() && done[1].output_token_ids == expectedTokens(prompt(3), 6), "mixed: decode lane tokens");
    check(done[2].ok() && done[2].output_token_ids == expectedTokens(prompt(40), 3), "mixed: chunked lane tokens");
    // Runner limit smaller than the budget: positions per call stay within it.
    FakeBackend kv2;
    FakeRunner m2;
    m2.spans = true;
    m2.max_batch = 10;
    IterationSchedulerRuntime s2(kv2, m2, {4, 64, 1 << 16, 16});
    check(s2.submit(req(5, 30, 2)).ok() && s2.submit(req(6, 30, 2)).ok(), "limit: accepted");
    auto d2 = byId(s2.drain());
    check(std::all_of(m2.span_calls.begin(), m2.span_calls.end(), [](std::size_t n) { return n <= 10; }),
          "limit: calls within the runner limit");
    check(d2[5].output_token_ids == expectedTokens(prompt(30), 2) && d2[6].output_token_ids == d2[5].output_token_ids,
          "limit: tokens");
}

}  // namespace

int main()
{
    singleRequest();
    for (bool spans : {false, true}) {
        concurrency(spans);
        dynamicJoin(spans);
        chunkedPrefill(spans);
        isolation(spans);
        stopAndPressure(spans);
    }
    admission();
    destructorReclaims();
    mixedSpans();
    if (g_failures == 0) std::cout << "generation and scheduler contracts passed\n";
    return g_failures == 0 ? 0 : 1;
}
