#pragma once

// TinyLlama-shaped model runner on MI355X behind the generation SPI
// (counterpart of createCudaTinyLlamaModelRunner, src/cuda/model/
// runner_factory.cpp:56-196, and the batched forward of src/cuda/model/
// runner.cpp:410-848).  Weights are seeded N(0, 0.02) fp16 (RMSNorm weights
// one), or loaded from a checkpoint archive described by a weight manifest.  One forward call takes spans: a
// decode step (one position) goes through a token transaction and the fused
// split-K decode kernel, a prompt chunk (several positions) through a
// PrefillChunk and the MFMA chunked-prefill kernel; the dense layers run on
// all positions of the call at once (rocBLAS GEMMs, fused RMSNorm / RoPE /
// SwiGLU / argmax kernels).

#include "kim-kv/engine/generation.h"
#include "kim-kv/hip/hip_status.h"
#include "kim-kv/model/weight_manifest.h"

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace kimkvcache {

struct HipModelRunnerConfig final {
    TinyLlamaConfig model{};
    std::uint64_t weight_seed{0};
    std::uint32_t max_positions{0};   // positions per forward call
    std::uint32_t max_spans{0};       // requests per forward call
};

class HipTinyLlamaRunner final : public GenerationModelRunner {
public:
    // The backend's layout must match the model (layers, KV heads, head
    // dimension, query heads); `stream` carries every launch.  Returns null
    // and sets *error on a shape mismatch or an allocation failure.
    static std::unique_ptr<HipTinyLlamaRunner> create(EngineKvBackend& kv, HipModelRunnerConfig const& config,
                                                      HipStream stream, std::string* error);
    // Weights from a checkpoint archive instead of the seed (the reference's
    // createCudaTinyLlamaModelRunner(kv, manifest_path, data_path, ...),
    // src/cuda/model/runner_factory.cpp:11-196): the manifest is loaded and
    // validated, every tensor range of the data file is checked against its
    // SHA-256, the model dimensions come from the manifest, and the tensors
    // are copied into the runner's fused q|k|v and gate|up matrices.
    static std::unique_ptr<HipTinyLlamaRunner> createFromArchive(EngineKvBackend& kv, std::string const& manifest_path,
                                                                 std::string const& data_path,
                                                                 std::uint32_t max_positions, std::uint32_t max_spans,
                                                                 HipStream stream, std::string* error);
    ~HipTinyLlamaRunner() override;

    TinyLlamaConfig generationConfig() const noexcept override;
    GenerationStepResult generationForwardToken(RequestId request_id, std::uint32_t token_id,
                                                std::uint32_t expected_position) override;
    GenerationBatchResult generationForwardBatch(std::vector<GenerationBatchItem> const& batch) override;
    std::uint32_t generationMaxBatchSize() const noexcept override;
    bool generationSupportsSpans() const noexcept override { return true; }
    GenerationBatchResult generationForwardSpans(std::vector<GenerationSpan> const& spans) override;

    // The same forward, also copying the fp32 logits after each span's last
    // position to host_logits ([spans.size()][vocabulary]) when non-null.
    GenerationBatchResult forwardSpans(std::vector<GenerationSpan> const& spans, float* host_logits);

    // Observation hook with no counterpart in the reference (its runner tests
    // compare generated tokens): after each forward -- the scheduler's
    // included -- that holds a span of request ids[k], the fp32 logits after
    // that span's last position are copied to rows + k * vocabulary,
    // positions[k] is set to that position and counts[k] is incremented.
    // The buffers are the caller's host memory and must stay valid while the
    // watch lasts; an empty id list (or a null buffer) ends it.  Not thread
    // safe, like the forward calls it observes.
    void watchLogits(std::vector<RequestId> ids, float* rows, std::uint32_t* positions, std::uint32_t* counts);

    std::uint64_t deviceWeightBytes() const noexcept;
    std::uint64_t deviceWorkspaceBytes() const noexcept;

    struct Impl;

private:
    explicit HipTinyLlamaRunner(std::unique_ptr<Impl> impl) noexcept;
    std::unique_ptr<Impl> impl_;
};

}  // namespace kimkvcache
