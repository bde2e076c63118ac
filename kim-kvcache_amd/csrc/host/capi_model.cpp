// C facade over the model runner and the iteration scheduler
// (include/kimkv_host.h, kimkv_runner_* / kimkv_scheduler_*).
#include "kimkv_host.h"

#include "capi_internal.h"
#include "kim-kv/engine/iteration_scheduler.h"
#include "kim-kv/hip/hip_model_runner.h"

#include <algorithm>
#include <cstring>
#include <memory>
#include <string>
#include <new>
#include <vector>

using namespace kimkvcache;

struct kimkv_runner {
    std::unique_ptr<HipTinyLlamaRunner> runner;
};

struct kimkv_scheduler {
    std::unique_ptr<IterationSchedulerRuntime> scheduler;
    std::vector<GenerationTerminal> delivered;
};

extern "C" {

kimkv_runner* kimkv_runner_create(kimkv_engine* e, const kimkv_model_config* model, uint64_t weight_seed,
                                  uint32_t max_positions, uint32_t max_spans, kimkv_stream_t stream)
{
    if (e == nullptr || model == nullptr) return nullptr;
    HipModelRunnerConfig c;
    c.model = TinyLlamaConfig{model->hidden_size,          model->intermediate_size, model->layer_count,
                              model->attention_head_count, model->kv_head_count,     model->head_dimension,
                              model->vocabulary_size,      model->max_position_embeddings,
                              model->bos_token_id,         model->eos_token_id,      model->rms_norm_epsilon,
                              model->rope_theta,           false};
    c.weight_seed = weight_seed;
    c.max_positions = max_positions;
    c.max_spans = max_spans;
    try {
        std::string error;
        std::unique_ptr<HipTinyLlamaRunner> r = HipTinyLlamaRunner::create(*e->backend, c, stream, &error);
        if (r == nullptr) return nullptr;
        return new kimkv_runner{std::move(r)};
    } catch (...) {
        return nullptr;
    }
}

kimkv_runner* kimkv_runner_create_from_archive(kimkv_engine* e, const char* manifest_path, const char* data_path,
                                               uint32_t max_positions, uint32_t max_spans, kimkv_stream_t stream,
                                               char* error, size_t error_capacity)
{
    if (error != nullptr && error_capacity != 0) error[0] = '\0';
    if (e == nullptr || manifest_path == nullptr || data_path == nullptr) return nullptr;
    std::string message;
    try {
        std::unique_ptr<HipTinyLlamaRunner> r = HipTinyLlamaRunner::createFromArchive(
            *e->backend, manifest_path, data_path, max_positions, max_spans, stream, &message);
        if (r != nullptr) return new kimkv_runner{std::move(r)};
    } catch (...) {
        message = "unexpected exception";
    }
    if (error != nullptr && error_capacity != 0) {
        std::size_t const n = std::min(message.size(), error_capacity - 1);
        std::memcpy(error, message.data(), n);
        error[n] = '\0';
    }
    return nullptr;
}

void kimkv_runner_destroy(kimkv_runner* r) { delete r; }
uint64_t kimkv_runner_weight_bytes(const kimkv_runner* r) { return r->runner->deviceWeightBytes(); }

int kimkv_runner_forward(kimkv_runner* r, uint32_t span_count, const uint64_t* request_ids,
                         const uint32_t* first_positions, const uint32_t* token_counts, const uint32_t* tokens,
                         uint32_t* next_tokens, int* step_ok, float* logits)
{
    try {
        std::vector<GenerationSpan> spans(span_count);
        std::size_t off = 0;
        for (uint32_t i = 0; i < span_count; ++i) {
            spans[i].request_id = request_ids[i];
            spans[i].first_position = first_positions[i];
            spans[i].token_ids.assign(tokens + off, tokens + off + token_counts[i]);
            off += token_counts[i];
        }
        GenerationBatchResult res = r->runner->forwardSpans(spans, logits);
        if (!res.success || res.steps.size() != span_count) return -1;
        for (uint32_t i = 0; i < span_count; ++i) {
            next_tokens[i] = res.steps[i].greedy_token_id;
            step_ok[i] = res.steps[i].success ? 1 : 0;
        }
        return 0;
    } catch (...) {
        return -1;
    }
}

int kimkv_runner_watch_logits(kimkv_runner* r, uint32_t count, const uint64_t* request_ids, float* rows,
                              uint32_t* positions, uint32_t* counts)
{
    if (r == nullptr || (count != 0 && (request_ids == nullptr || rows == nullptr || positions == nullptr
                                        || counts == nullptr))) {
        return -1;
    }
    try {
        r->runner->watchLogits(std::vector<RequestId>(request_ids, request_ids + count), rows, positions, counts);
        return 0;
    } catch (...) {
        return -1;
    }
}

kimkv_scheduler* kimkv_scheduler_create(kimkv_engine* e, kimkv_runner* r, const kimkv_scheduler_config* config)
{
    if (e == nullptr || r == nullptr || config == nullptr) return nullptr;
    try {
        IterationSchedulerConfig c{config->max_active_requests, config->max_batched_tokens, config->max_kv_tokens,
                                   config->prefill_chunk_size};
        auto s = std::make_unique<IterationSchedulerRuntime>(*e->backend, *r->runner, c);
        return new kimkv_scheduler{std::move(s), {}};
    } catch (...) {
        return nullptr;
    }
}

void kimkv_scheduler_destroy(kimkv_scheduler* s) { delete s; }

int kimkv_scheduler_submit(kimkv_scheduler* s, uint64_t request_id, const uint32_t* prompt, uint32_t prompt_length,
                           uint32_t max_new_tokens, int64_t eos_token_id)
{
    try {
        GenerationRequest req;
        req.request_id = request_id;
        if (prompt != nullptr) req.prompt_token_ids.assign(prompt, prompt + prompt_length);
        req.sampling.max_new_tokens = max_new_tokens;
        if (eos_token_id >= 0) req.sampling.eos_token_id = static_cast<std::uint32_t>(eos_token_id);
        return static_cast<int>(s->scheduler->submit(std::move(req)).error);
    } catch (...) {
        return static_cast<int>(SchedulerAdmissionError::InternalError);
    }
}

int kimkv_scheduler_cancel(kimkv_scheduler* s, uint64_t request_id) { return s->scheduler->cancel(request_id) ? 1 : 0; }

void kimkv_scheduler_run_iteration(kimkv_scheduler* s, kimkv_iteration_result* out)
{
    SchedulerIterationResult const r = s->scheduler->runIteration();
    if (out != nullptr) {
        *out = kimkv_iteration_result{r.iteration, r.model_forward_tokens, r.model_forward_batches, r.prefill_tokens,
                                      r.decode_tokens, r.terminals_produced};
    }
}

static uint32_t deliver(kimkv_scheduler* s, std::vector<GenerationTerminal> t)
{
    for (GenerationTerminal& x : t) s->delivered.push_back(std::move(x));
    return static_cast<uint32_t>(s->delivered.size());
}

uint32_t kimkv_scheduler_drain(kimkv_scheduler* s) { return deliver(s, s->scheduler->drain()); }
uint32_t kimkv_scheduler_collect(kimkv_scheduler* s) { return deliver(s, s->scheduler->takeTerminals()); }

int kimkv_scheduler_terminal(const kimkv_scheduler* s, uint32_t index, kimkv_terminal_info* info, uint32_t* tokens,
                             uint32_t capacity)
{
    if (index >= s->delivered.size()) return -1;
    GenerationTerminal const& t = s->delivered[index];
    if (info != nullptr) {
        *info = kimkv_terminal_info{t.request_id,         static_cast<uint32_t>(t.reason), static_cast<uint32_t>(t.error),
                                    t.usage.prompt_tokens, t.usage.completion_tokens,      t.metrics.ttft_ns,
                                    t.metrics.tpot_ns,     t.metrics.e2e_ns};
    }
    uint32_t const n = static_cast<uint32_t>(t.output_token_ids.size());
    if (tokens != nullptr) std::copy_n(t.output_token_ids.begin(), std::min(n, capacity), tokens);
    return static_cast<int>(n);
}

void kimkv_scheduler_clear_terminals(kimkv_scheduler* s) { s->delivered.clear(); }
int kimkv_scheduler_idle(const kimkv_scheduler* s) { return s->scheduler->idle() ? 1 : 0; }

}  // extern "C"
