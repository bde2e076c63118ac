// TinyLlama runner over the HIP engine backend (counterpart of
// src/cuda/model/runner.cpp:410-848 and runner_factory.cpp:56-196).
//
// One forward call = one iteration's spans.  Per call: token ids / positions
// / last-row indices go up in one staged copy; decode steps reserve token
// transactions in one batch, prompt chunks open PrefillChunks; then per layer
//   RMSNorm -> QKV GEMM -> RoPE + split -> K/V writes (one append launch for
//   the decode lanes, one for the chunks) -> attention (one decode launch,
//   one chunked-prefill launch) -> O GEMM (+ residual) -> RMSNorm ->
//   gate|up GEMM -> SwiGLU -> down GEMM (+ residual);
// finally RMSNorm of each span's last row, the LM head (fp32 logits) and the
// argmax.  Commits / finishes are the call's completion point.
#include "kim-kv/hip/hip_model_runner.h"

#include "kim-kv/hip/hip_engine_kv_backend.h"
#include "kimkv_hip.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <fstream>
#include <new>
#include <utility>

namespace kimkvcache {

namespace {

// N(0, 0.02) from the synthetic generator (std 2 / sqrt(3)): scale = 0.02 * sqrt(3) / 2.
constexpr float kWeightScale = 0.017320508f;
constexpr std::uint16_t kOneF16 = 0x3C00;

// Row ids of the seeded weights: tensor `kind` of layer `layer` (layer ==
// layer_count for the embedding, final norm and LM head) starts at row
// (layer + 1) << 40 | kind << 32.
enum WeightKind : std::uint32_t { kQ = 1, kK, kV, kO, kGate, kUp, kDown, kEmbed, kHead };

std::uint64_t weightRow(std::uint32_t layer, std::uint32_t kind)
{
    return (static_cast<std::uint64_t>(layer + 1) << 40) | (static_cast<std::uint64_t>(kind) << 32);
}

std::size_t align256(std::size_t n) { return (n + 255) & ~std::size_t{255}; }

// Row counts of the per-layer GEMMs are padded to a multiple of this, so a
// handful of tuned problem sizes covers every forward.
constexpr std::uint32_t kGemmRowQuantum = 128;

}  // namespace

struct HipTinyLlamaRunner::Impl {
    EngineKvBackend* kv{nullptr};
    HipModelRunnerConfig cfg{};
    HipStream stream{nullptr};
    std::uint32_t QD{0}, KD{0}, W_qkv{0};
    std::size_t ws_lane{0};   // decode split-K workspace per lane
    std::uint32_t gemm_cap{0};   // activation rows: max_positions rounded up to kGemmRowQuantum

    // Device memory: one block for weights, one for activations.
    void* weights{nullptr};
    std::uint64_t weight_bytes{0};
    void* work{nullptr};
    std::uint64_t work_bytes{0};
    void* pinned{nullptr};   // ids / positions / last rows up, tokens down

    struct Layer {
        std::uint16_t *ln1, *wqkv, *wo, *ln2, *wgu, *wdown;
    };
    std::vector<Layer> layers;
    std::uint16_t *embed{nullptr}, *final_norm{nullptr}, *head{nullptr};

    // Activations.
    std::uint16_t *x{nullptr}, *h{nullptr}, *qkv{nullptr}, *q{nullptr}, *k{nullptr}, *v{nullptr}, *attn{nullptr},
        *gu{nullptr}, *act{nullptr}, *hf{nullptr};
    float* logits{nullptr};
    std::uint32_t *d_ids{nullptr}, *d_pos{nullptr}, *d_last{nullptr}, *d_tokens{nullptr};
    std::uint8_t* decode_ws{nullptr};
    DevicePagedDecodeBatchItem* d_items{nullptr};

    // The decode lanes' token transactions run on their own stream, so a
    // layer's decode attention runs beside its chunked-prefill attention
    // (they read different requests' pages) and fills the compute units the
    // prefill launch's last workgroups leave idle.  Per layer the decode
    // stream waits for the main stream's q/k/v (qkv_ready) and the main
    // stream waits for the decode outputs (decode_done) before the output
    // projection.
    HipStream decode_stream{nullptr};
    void* qkv_ready{nullptr};
    void* decode_done{nullptr};

    // Watched requests (watchLogits): their spans' logits rows go to the
    // caller's host buffers after each forward.
    std::vector<RequestId> watch_ids;
    float* watch_rows{nullptr};
    std::uint32_t* watch_positions{nullptr};
    std::uint32_t* watch_counts{nullptr};

    ~Impl()
    {
        if (decode_stream) {
            static_cast<void>(kimkv_stream_synchronize(decode_stream));
            kimkv_stream_destroy(decode_stream);
        }
        if (qkv_ready) kimkv_event_destroy(qkv_ready);
        if (decode_done) kimkv_event_destroy(decode_done);
        if (weights) kimkv_device_free(weights);
        if (work) kimkv_device_free(work);
        if (pinned) kimkv_host_free_pinned(pinned);
    }

    bool allocate(std::string* error)
    {
        if (kimkv_stream_create(&decode_stream) != KIMKV_OK
            || kimkv_event_create(&qkv_ready, KIMKV_EVENT_ORDER_ONLY) != KIMKV_OK
            || kimkv_event_create(&decode_done, KIMKV_EVENT_ORDER_ONLY) != KIMKV_OK) {
            if (error) *error = "decode stream creation failed";
            return false;
        }
        TinyLlamaConfig const& m = cfg.model;
        std::uint64_t const H = m.hidden_size, I = m.intermediate_size, V = m.vocabulary_size;
        std::uint64_t per_layer = 0;
        per_layer += align256(H * 2) * 2;                              // ln1, ln2
        per_layer += align256(std::uint64_t{W_qkv} * H * 2);           // q|k|v
        per_layer += align256(H * H * 2);                              // o
        per_layer += align256(2 * I * H * 2);                          // gate|up
        per_layer += align256(H * I * 2);                              // down
        weight_bytes = per_layer * m.layer_count + align256(V * H * 2) * 2 + align256(H * 2);
        if (kimkv_device_malloc(&weights, weight_bytes) != KIMKV_OK) {
            if (error) *error = "weight allocation failed";
            return false;
        }
        auto* p = static_cast<std::uint8_t*>(weights);
        auto take = [&p](std::uint64_t bytes) {
            auto* r = reinterpret_cast<std::uint16_t*>(p);
            p += align256(bytes);
            return r;
        };
        layers.resize(m.layer_count);
        for (Layer& L : layers) {
            L.ln1 = take(H * 2);
            L.wqkv = take(std::uint64_t{W_qkv} * H * 2);
            L.wo = take(H * H * 2);
            L.ln2 = take(H * 2);
            L.wgu = take(2 * I * H * 2);
            L.wdown = take(H * I * 2);
        }
        embed = take(V * H * 2);
        final_norm = take(H * 2);
        head = take(V * H * 2);

        gemm_cap = (cfg.max_positions + kGemmRowQuantum - 1) / kGemmRowQuantum * kGemmRowQuantum;
        std::uint64_t const P = gemm_cap, S = cfg.max_spans;
        std::uint64_t sizes[] = {
            P * H * 2, P * H * 2, P * W_qkv * 2, P * QD * 2, P * KD * 2, P * KD * 2, P * QD * 2,
            P * 2 * I * 2, P * I * 2, S * H * 2, S * V * 4, P * 4, P * 4, S * 4, S * 4,
            S * ws_lane, S * sizeof(DevicePagedDecodeBatchItem)};
        work_bytes = 0;
        for (std::uint64_t s : sizes) work_bytes += align256(s);
        if (kimkv_device_malloc(&work, work_bytes) != KIMKV_OK) {
            if (error) *error = "workspace allocation failed";
            return false;
        }
        p = static_cast<std::uint8_t*>(work);
        x = take(sizes[0]);
        h = take(sizes[1]);
        qkv = take(sizes[2]);
        q = take(sizes[3]);
        k = take(sizes[4]);
        v = take(sizes[5]);
        attn = take(sizes[6]);
        gu = take(sizes[7]);
        act = take(sizes[8]);
        hf = take(sizes[9]);
        logits = reinterpret_cast<float*>(take(sizes[10]));
        d_ids = reinterpret_cast<std::uint32_t*>(take(sizes[11]));
        d_pos = reinterpret_cast<std::uint32_t*>(take(sizes[12]));
        d_last = reinterpret_cast<std::uint32_t*>(take(sizes[13]));
        d_tokens = reinterpret_cast<std::uint32_t*>(take(sizes[14]));
        decode_ws = reinterpret_cast<std::uint8_t*>(take(sizes[15]));
        d_items = reinterpret_cast<DevicePagedDecodeBatchItem*>(take(sizes[16]));
        if (kimkv_host_malloc_pinned(&pinned, (2 * P + 2 * S) * 4) != KIMKV_OK) {
            if (error) *error = "pinned staging allocation failed";
            return false;
        }
        return true;
    }

    // Picks the GEMM algorithm of every padded row count the forward can use
    // (multiples of kGemmRowQuantum up to gemm_cap) on the activation
    // buffers, timing each candidate over all layers' weights.
    bool tuneGemms()
    {
        TinyLlamaConfig const& m = cfg.model;
        std::vector<std::uint16_t const*> wqkv, wo, wgu, wdown;
        for (Layer const& L : layers) {
            wqkv.push_back(L.wqkv);
            wo.push_back(L.wo);
            wgu.push_back(L.wgu);
            wdown.push_back(L.wdown);
        }
        auto const n = static_cast<std::uint32_t>(layers.size());
        bool ok = true;
        for (std::uint32_t g = kGemmRowQuantum; g <= gemm_cap && ok; g += kGemmRowQuantum) {
            ok = kimkv_linear_tune(h, g, m.hidden_size, wqkv.data(), n, W_qkv, qkv, 0, 0.0f, stream) == KIMKV_OK
                && kimkv_linear_tune(attn, g, m.hidden_size, wo.data(), n, m.hidden_size, x, 0, 1.0f, stream) == KIMKV_OK
                && kimkv_linear_tune(h, g, m.hidden_size, wgu.data(), n, 2 * m.intermediate_size, gu, 0, 0.0f, stream)
                    == KIMKV_OK
                && kimkv_linear_tune(act, g, m.intermediate_size, wdown.data(), n, m.hidden_size, x, 0, 1.0f, stream)
                    == KIMKV_OK;
        }
        return ok && kimkv_stream_synchronize(stream) == KIMKV_OK;
    }

    bool initWeights()
    {
        TinyLlamaConfig const& m = cfg.model;
        std::uint64_t const H = m.hidden_size, I = m.intermediate_size, V = m.vocabulary_size;
        std::uint64_t const seed = cfg.weight_seed;
        bool ok = true;
        auto fill = [&](std::uint16_t* dst, std::uint64_t rows, std::uint64_t cols, std::uint64_t row0) {
            ok = ok && kimkv_fill_rows_scaled(dst, rows * cols, seed, row0, static_cast<std::uint32_t>(cols),
                                              kWeightScale, stream) == KIMKV_OK;
        };
        auto ones = [&](std::uint16_t* dst, std::uint64_t n) {
            ok = ok && kimkv_fill_f16(dst, n, kOneF16, stream) == KIMKV_OK;
        };
        for (std::uint32_t l = 0; l < m.layer_count; ++l) {
            Layer const& L = layers[l];
            ones(L.ln1, H);
            ones(L.ln2, H);
            fill(L.wqkv, QD, H, weightRow(l, kQ));
            fill(L.wqkv + std::uint64_t{QD} * H, KD, H, weightRow(l, kK));
            fill(L.wqkv + std::uint64_t{QD + KD} * H, KD, H, weightRow(l, kV));
            fill(L.wo, H, H, weightRow(l, kO));
            fill(L.wgu, I, H, weightRow(l, kGate));
            fill(L.wgu + I * H, I, H, weightRow(l, kUp));
            fill(L.wdown, H, I, weightRow(l, kDown));
        }
        fill(embed, V, H, weightRow(m.layer_count, kEmbed));
        ones(final_norm, H);
        fill(head, V, H, weightRow(m.layer_count, kHead));
        return ok && kimkv_stream_synchronize(stream) == KIMKV_OK;
    }

    // Copies every tensor of a validated archive to its place in the weight
    // block (fused q|k|v and gate|up rows), through a pinned staging buffer
    // in pieces of at most kStagePiece bytes.
    bool loadArchive(WeightManifest const& manifest, std::string const& data_path, std::string* error)
    {
        TinyLlamaConfig const& m = cfg.model;
        std::uint64_t const H = m.hidden_size, I = m.intermediate_size;
        auto target = [&](std::string const& name) -> std::uint16_t* {
            if (name == "model.embed_tokens.weight") return embed;
            if (name == "model.norm.weight") return final_norm;
            if (name == "lm_head.weight") return head;
            std::string const prefix = "model.layers.";
            if (name.compare(0, prefix.size(), prefix) != 0) return nullptr;
            std::size_t dot = name.find('.', prefix.size());
            if (dot == std::string::npos) return nullptr;
            std::uint32_t l = 0;
            for (std::size_t i = prefix.size(); i < dot; ++i) {
                if (name[i] < '0' || name[i] > '9') return nullptr;
                l = l * 10 + static_cast<std::uint32_t>(name[i] - '0');
                if (l >= layers.size()) return nullptr;
            }
            Layer const& L = layers[l];
            std::string const part = name.substr(dot + 1);
            if (part == "input_layernorm.weight") return L.ln1;
            if (part == "post_attention_layernorm.weight") return L.ln2;
            if (part == "self_attn.q_proj.weight") return L.wqkv;
            if (part == "self_attn.k_proj.weight") return L.wqkv + std::uint64_t{QD} * H;
            if (part == "self_attn.v_proj.weight") return L.wqkv + std::uint64_t{QD + KD} * H;
            if (part == "self_attn.o_proj.weight") return L.wo;
            if (part == "mlp.gate_proj.weight") return L.wgu;
            if (part == "mlp.up_proj.weight") return L.wgu + I * H;
            if (part == "mlp.down_proj.weight") return L.wdown;
            return nullptr;
        };
        constexpr std::size_t kStagePiece = std::size_t{32} << 20;
        void* stage = nullptr;
        if (kimkv_host_malloc_pinned(&stage, 2 * kStagePiece) != KIMKV_OK) {
            if (error) *error = "pinned staging allocation failed";
            return false;
        }
        std::ifstream in(data_path, std::ios::binary);
        bool ok = static_cast<bool>(in);
        int half = 0;
        void* pending[2] = {nullptr, nullptr};   // an event per staging half while its copy is in flight
        for (WeightTensorDescriptor const& t : manifest.tensors) {
            std::uint16_t* dst = target(t.name);
            if (!ok || dst == nullptr) {
                ok = false;
                break;
            }
            in.seekg(static_cast<std::streamoff>(t.offset));
            for (std::uint64_t done = 0; ok && done < t.byte_size;) {
                auto const n = static_cast<std::size_t>(std::min<std::uint64_t>(kStagePiece, t.byte_size - done));
                auto* buf = static_cast<char*>(stage) + half * kStagePiece;
                if (pending[half] != nullptr) {   // the copy out of this half must finish before it is refilled
                    ok = kimkv_event_synchronize(pending[half]) == KIMKV_OK;
                    kimkv_event_destroy(pending[half]);
                    pending[half] = nullptr;
                }
                in.read(buf, static_cast<std::streamsize>(n));
                ok = ok && in.gcount() == static_cast<std::streamsize>(n)
                    && kimkv_memcpy_h2d_async(reinterpret_cast<char*>(dst) + done, buf, n, stream) == KIMKV_OK
                    && kimkv_event_create(&pending[half], 0) == KIMKV_OK
                    && kimkv_event_record(pending[half], stream) == KIMKV_OK;
                done += n;
                half ^= 1;
            }
        }
        ok = kimkv_stream_synchronize(stream) == KIMKV_OK && ok;
        for (void* e : pending) {
            if (e != nullptr) kimkv_event_destroy(e);
        }
        kimkv_host_free_pinned(stage);
        if (!ok && error) *error = "reading the weight archive into device memory failed";
        return ok;
    }

    GenerationBatchResult forward(std::vector<GenerationSpan> const& spans, float* host_logits);
};

GenerationBatchResult HipTinyLlamaRunner::Impl::forward(std::vector<GenerationSpan> const& spans, float* host_logits)
{
    GenerationBatchResult result;
    TinyLlamaConfig const& m = cfg.model;
    std::size_t const S = spans.size();
    if (S == 0 || S > cfg.max_spans) {
        result.detail = "span count is zero or above the runner's max_spans";
        return result;
    }
    std::uint32_t P = 0;
    for (GenerationSpan const& s : spans) {
        if (s.token_ids.empty() || s.request_id == kInvalidRequestId) {
            result.detail = "span without tokens or request id";
            return result;
        }
        for (std::uint32_t t : s.token_ids) {
            if (t >= m.vocabulary_size) {
                result.detail = "token id outside the vocabulary";
                return result;
            }
        }
        if (static_cast<std::uint64_t>(s.first_position) + s.token_ids.size() > m.max_position_embeddings) {
            result.detail = "span runs past max_position_embeddings";
            return result;
        }
        P += static_cast<std::uint32_t>(s.token_ids.size());
    }
    if (P > cfg.max_positions) {
        result.detail = "span positions exceed the runner's max_positions";
        return result;
    }

    // Host staging: ids[P], positions[P], last rows[S].
    auto* st = static_cast<std::uint32_t*>(pinned);
    std::uint32_t* ids = st;
    std::uint32_t* pos = st + cfg.max_positions;
    std::uint32_t* last = st + 2 * cfg.max_positions;
    std::uint32_t* tokens_out = last + cfg.max_spans;
    std::vector<std::uint32_t> first_row(S);
    std::uint32_t r = 0;
    for (std::size_t i = 0; i < S; ++i) {
        first_row[i] = r;
        for (std::size_t t = 0; t < spans[i].token_ids.size(); ++t, ++r) {
            ids[r] = spans[i].token_ids[t];
            pos[r] = spans[i].first_position + static_cast<std::uint32_t>(t);
        }
        last[i] = r - 1;
    }
    bool ok = kimkv_memcpy_h2d_async(d_ids, ids, P * 4ull, stream) == KIMKV_OK
        && kimkv_memcpy_h2d_async(d_pos, pos, P * 4ull, stream) == KIMKV_OK
        && kimkv_memcpy_h2d_async(d_last, last, S * 4ull, stream) == KIMKV_OK;

    // The four per-layer GEMMs run on G >= P rows (P rounded up to the tuned
    // quantum); rows P..G-1 of their inputs and outputs are scratch that no
    // other kernel reads.
    std::uint32_t const G = std::min<std::uint32_t>((P + kGemmRowQuantum - 1) / kGemmRowQuantum * kGemmRowQuantum,
                                                    gemm_cap);
    // Layer l up to its K/V: RMSNorm, QKV projection, RoPE.  The embedding and
    // layer 0's part go to the device before the token reservations and chunk
    // begins below, so the device works while the host does those.
    auto pre_attention = [&](Layer const& L) {
        return kimkv_model_rmsnorm(x, nullptr, P, L.ln1, m.hidden_size, m.rms_norm_epsilon, h, stream) == KIMKV_OK
            && kimkv_linear(h, G, m.hidden_size, L.wqkv, W_qkv, qkv, 0, 0.0f, stream) == KIMKV_OK
            && kimkv_model_rope_split(qkv, d_pos, P, m.attention_head_count, m.kv_head_count, m.head_dimension,
                                      m.rope_theta, q, k, v, stream) == KIMKV_OK;
    };
    ok = ok && kimkv_model_embed(embed, d_ids, P, m.hidden_size, x, stream) == KIMKV_OK && pre_attention(layers[0]);

    // KV side: token transactions for single positions, prefill chunks for the rest.
    std::vector<GenerationStepResult> steps(S, GenerationStepResult{true, 0, {}});
    std::vector<std::size_t> dec, pre;
    for (std::size_t i = 0; i < S; ++i) (spans[i].token_ids.size() == 1 ? dec : pre).push_back(i);
    std::vector<ReserveTokenRequest> reqs(dec.size());
    std::vector<TokenReserveResult> reserved(dec.size());
    for (std::size_t j = 0; j < dec.size(); ++j) {
        reqs[j] = ReserveTokenRequest{spans[dec[j]].request_id, spans[dec[j]].first_position, decode_stream};
    }
    if (!dec.empty() && !reserveTokenBatch(*kv, reqs.data(), reqs.size(), reserved.data())) {
        for (std::size_t j = 0; j < dec.size(); ++j) reserved[j].status = {EngineKvError::InvalidArgument};
    }
    auto fail = [&steps](std::size_t i, std::string text) {
        if (steps[i].success) steps[i] = GenerationStepResult{false, 0, std::move(text)};
    };
    for (std::size_t j = 0; j < dec.size(); ++j) {
        if (!reserved[j].ok()) fail(dec[j], "token reservation failed: " + std::string(toString(reserved[j].status.error)));
    }
    std::vector<PrefillChunk> chunks(pre.size());
    for (std::size_t j = 0; j < pre.size(); ++j) {
        GenerationSpan const& s = spans[pre[j]];
        PrefillChunkResult c = beginPrefillChunk(*kv, s.request_id, s.first_position,
                                                 static_cast<std::uint32_t>(s.token_ids.size()), stream);
        if (c.ok()) {
            chunks[j] = std::move(c.chunk);
        } else {
            fail(pre[j], "prefill chunk refused: " + std::string(toString(c.status.error)));
        }
    }

    float const scale = 1.0f / std::sqrt(static_cast<float>(m.head_dimension));
    std::vector<LayerKvWriteBatchItem> wr;
    std::vector<PagedDecodeBatchItem> at;
    std::vector<DevicePagedDecodeBatchItem> at_host(dec.size());
    std::vector<PrefillChunk*> live_chunks;
    std::vector<std::size_t> live_pre;
    std::vector<KvScalar const*> pk, pv, pq;
    std::vector<KvScalar*> po;
    std::vector<EngineKvStatus> pst;

    for (std::uint32_t l = 0; l < m.layer_count && ok; ++l) {
        Layer const& L = layers[l];
        if (l > 0) ok = pre_attention(L);
        // The decode stream starts the layer once its q/k/v rows exist.
        ok = ok && kimkv_event_record(qkv_ready, stream) == KIMKV_OK
            && kimkv_stream_wait_event(decode_stream, qkv_ready) == KIMKV_OK;
        if (!ok) break;
        // Writes.
        wr.clear();
        std::vector<std::size_t> wr_owner;
        for (std::size_t j = 0; j < dec.size(); ++j) {
            if (!steps[dec[j]].success) continue;
            std::uint64_t const row = first_row[dec[j]];
            LayerKvWriteBatchItem it;
            it.transaction = &reserved[j].transaction;
            it.write = LayerKvWrite{l, k + row * KD, v + row * KD};
            wr.push_back(it);
            wr_owner.push_back(dec[j]);
        }
        if (!wr.empty()) {
            LayerKvWriteBatch b{wr.data(), wr.size()};
            writeLayerBatch(b);
        }
        live_chunks.clear();
        live_pre.clear();
        pk.clear();
        pv.clear();
        for (std::size_t j = 0; j < pre.size(); ++j) {
            if (!steps[pre[j]].success) continue;
            std::uint64_t const row = first_row[pre[j]];
            live_chunks.push_back(&chunks[j]);
            live_pre.push_back(pre[j]);
            pk.push_back(k + row * KD);
            pv.push_back(v + row * KD);
        }
        pst.assign(live_chunks.size(), EngineKvStatus{});
        if (!live_chunks.empty()) {
            writePrefillBatch(live_chunks.data(), live_chunks.size(), l, pk.data(), pv.data(), pst.data());
        }
        for (std::size_t w = 0; w < wr.size(); ++w) {
            if (!wr[w].status.ok()) fail(wr_owner[w], "K/V write failed: " + std::string(toString(wr[w].status.error)));
        }
        for (std::size_t c = 0; c < live_pre.size(); ++c) {
            if (!pst[c].ok()) fail(live_pre[c], "chunk K/V write failed: " + std::string(toString(pst[c].error)));
        }
        // Attention.
        at.clear();
        std::vector<std::size_t> at_owner;
        for (std::size_t j = 0; j < dec.size(); ++j) {
            if (!steps[dec[j]].success) continue;
            std::uint64_t const row = first_row[dec[j]];
            PagedDecodeBatchItem it;
            it.transaction = &reserved[j].transaction;
            it.request = PagedDecodeRequest{l, q + row * QD, attn + row * QD, decode_ws + at.size() * ws_lane, ws_lane,
                                            scale};
            at.push_back(it);
            at_owner.push_back(dec[j]);
        }
        if (!at.empty()) {
            PagedDecodeBatch b{at.data(), at.size(), at_host.data(), d_items, dec.size()};
            attendLayerBatch(b);
            for (std::size_t a = 0; a < at.size(); ++a) {
                if (!at[a].status.ok()) fail(at_owner[a], "decode attention failed: " + std::string(toString(at[a].status.error)));
            }
        }
        live_chunks.clear();
        live_pre.clear();
        pq.clear();
        po.clear();
        for (std::size_t j = 0; j < pre.size(); ++j) {
            if (!steps[pre[j]].success) continue;
            std::uint64_t const row = first_row[pre[j]];
            live_chunks.push_back(&chunks[j]);
            live_pre.push_back(pre[j]);
            pq.push_back(q + row * QD);
            po.push_back(attn + row * QD);
        }
        pst.assign(live_chunks.size(), EngineKvStatus{});
        if (!live_chunks.empty()) {
            attendPrefillBatch(live_chunks.data(), live_chunks.size(), l, pq.data(), po.data(), scale, pst.data());
            for (std::size_t c = 0; c < live_pre.size(); ++c) {
                if (!pst[c].ok()) fail(live_pre[c], "chunk attention failed: " + std::string(toString(pst[c].error)));
            }
        }
        // The decode lanes' attention rows are in attn before the output projection reads them.
        ok = kimkv_event_record(decode_done, decode_stream) == KIMKV_OK
            && kimkv_stream_wait_event(stream, decode_done) == KIMKV_OK;
        // Output projection + residual, MLP + residual.
        ok = ok && kimkv_linear(attn, G, m.hidden_size, L.wo, m.hidden_size, x, 0, 1.0f, stream) == KIMKV_OK
            && kimkv_model_rmsnorm(x, nullptr, P, L.ln2, m.hidden_size, m.rms_norm_epsilon, h, stream) == KIMKV_OK
            && kimkv_linear(h, G, m.hidden_size, L.wgu, 2 * m.intermediate_size, gu, 0, 0.0f, stream) == KIMKV_OK
            && kimkv_model_swiglu(gu, P, m.intermediate_size, act, stream) == KIMKV_OK
            && kimkv_linear(act, G, m.intermediate_size, L.wdown, m.hidden_size, x, 0, 1.0f, stream) == KIMKV_OK;
    }
    ok = ok && kimkv_model_rmsnorm(x, d_last, static_cast<std::uint32_t>(S), final_norm, m.hidden_size,
                                   m.rms_norm_epsilon, hf, stream) == KIMKV_OK
        && kimkv_linear(hf, static_cast<std::uint32_t>(S), m.hidden_size, head, m.vocabulary_size, logits, 1, 0.0f,
                        stream) == KIMKV_OK
        && kimkv_model_argmax(logits, static_cast<std::uint32_t>(S), m.vocabulary_size, d_tokens, stream) == KIMKV_OK
        && kimkv_memcpy_d2h_async(tokens_out, d_tokens, S * 4ull, stream) == KIMKV_OK;
    if (ok && host_logits != nullptr) {
        ok = kimkv_memcpy_d2h_async(host_logits, logits, S * std::uint64_t{m.vocabulary_size} * 4, stream) == KIMKV_OK;
    }
    // (watch slot, span) pairs of watched requests; rows copied here, the
    // positions and counts set once the forward has succeeded.
    std::vector<std::pair<std::size_t, std::size_t>> watched;
    for (std::size_t i = 0; ok && i < S && !watch_ids.empty(); ++i) {
        for (std::size_t k = 0; k < watch_ids.size(); ++k) {
            if (watch_ids[k] != spans[i].request_id) continue;
            watched.emplace_back(k, i);
            ok = kimkv_memcpy_d2h_async(watch_rows + k * std::uint64_t{m.vocabulary_size},
                                        logits + i * std::uint64_t{m.vocabulary_size},
                                        std::uint64_t{m.vocabulary_size} * 4, stream) == KIMKV_OK;
        }
    }

    // Completion: commit / finish (each waits for its work), then the stream.
    for (std::size_t j = 0; j < dec.size(); ++j) {
        if (!reserved[j].transaction.valid()) continue;
        if (steps[dec[j]].success && ok) {
            EngineKvStatus const c = reserved[j].transaction.commit();
            if (!c.ok()) fail(dec[j], "commit failed: " + std::string(toString(c.error)));
        } else {
            static_cast<void>(reserved[j].transaction.rollback());
        }
    }
    for (std::size_t j = 0; j < pre.size(); ++j) {
        if (!chunks[j].valid()) continue;
        EngineKvStatus const f = chunks[j].finish();
        if (!f.ok()) fail(pre[j], "prefill chunk finish failed: " + std::string(toString(f.error)));
    }
    if (kimkv_stream_synchronize(stream) != KIMKV_OK) ok = false;
    if (kimkv_stream_synchronize(decode_stream) != KIMKV_OK) ok = false;
    if (!ok) {
        result.detail = "device submission failed in the model forward";
        return result;
    }
    for (std::size_t i = 0; i < S; ++i) {
        if (steps[i].success) steps[i].greedy_token_id = tokens_out[i];
    }
    for (auto const& [k, i] : watched) {
        if (!steps[i].success) continue;
        watch_positions[k] = spans[i].first_position + static_cast<std::uint32_t>(spans[i].token_ids.size()) - 1;
        ++watch_counts[k];
    }
    result.steps = std::move(steps);
    result.success = true;
    return result;
}

// ---- public surface ---------------------------------------------------------------------

std::unique_ptr<HipTinyLlamaRunner> HipTinyLlamaRunner::create(EngineKvBackend& kv, HipModelRunnerConfig const& config,
                                                               HipStream stream, std::string* error)
{
    TinyLlamaConfig const& m = config.model;
    EngineKvConfig const e = kv.config();
    if (!m.valid() || config.max_positions == 0 || config.max_spans == 0) {
        if (error) *error = "invalid model or runner configuration";
        return nullptr;
    }
    if (e.kv_layout.layer_count != m.layer_count || e.kv_layout.kv_head_count != m.kv_head_count
        || e.kv_layout.head_dimension != m.head_dimension || e.query_head_count != m.attention_head_count) {
        if (error) *error = "KV backend layout does not match the model";
        return nullptr;
    }
    auto impl = std::make_unique<Impl>();
    impl->kv = &kv;
    impl->cfg = config;
    impl->stream = stream;
    impl->QD = m.attention_head_count * m.head_dimension;
    impl->KD = m.kv_head_count * m.head_dimension;
    impl->W_qkv = impl->QD + 2 * impl->KD;
    impl->ws_lane = (e.attention_workspace_bytes + 255) & ~std::size_t{255};
    if (!impl->allocate(error)) return nullptr;
    if (!impl->initWeights()) {
        if (error) *error = "weight initialisation failed";
        return nullptr;
    }
    if (!impl->tuneGemms()) {
        if (error) *error = "GEMM algorithm selection failed";
        return nullptr;
    }
    return std::unique_ptr<HipTinyLlamaRunner>(new HipTinyLlamaRunner(std::move(impl)));
}

std::unique_ptr<HipTinyLlamaRunner> HipTinyLlamaRunner::createFromArchive(EngineKvBackend& kv,
                                                                          std::string const& manifest_path,
                                                                          std::string const& data_path,
                                                                          std::uint32_t max_positions,
                                                                          std::uint32_t max_spans, HipStream stream,
                                                                          std::string* error)
{
    WeightManifestLoadResult loaded = loadWeightManifest(manifest_path);
    if (!loaded.ok()) {
        if (error) *error = "weight manifest: " + std::string(toString(loaded.status.error)) + ": " + loaded.status.detail;
        return nullptr;
    }
    WeightManifestStatus const data = validateWeightDataFile(loaded.manifest, data_path);
    if (!data.ok()) {
        if (error) *error = "weight archive: " + std::string(toString(data.error)) + ": " + data.detail;
        return nullptr;
    }
    TinyLlamaConfig const& m = loaded.manifest.config;
    EngineKvConfig const e = kv.config();
    if (max_positions == 0 || max_spans == 0) {
        if (error) *error = "invalid runner configuration";
        return nullptr;
    }
    if (e.kv_layout.layer_count != m.layer_count || e.kv_layout.kv_head_count != m.kv_head_count
        || e.kv_layout.head_dimension != m.head_dimension || e.query_head_count != m.attention_head_count) {
        if (error) *error = "KV backend layout does not match the model manifest";
        return nullptr;
    }
    auto impl = std::make_unique<Impl>();
    impl->kv = &kv;
    impl->cfg = HipModelRunnerConfig{m, 0, max_positions, max_spans};
    impl->stream = stream;
    impl->QD = m.attention_head_count * m.head_dimension;
    impl->KD = m.kv_head_count * m.head_dimension;
    impl->W_qkv = impl->QD + 2 * impl->KD;
    impl->ws_lane = (e.attention_workspace_bytes + 255) & ~std::size_t{255};
    if (!impl->allocate(error) || !impl->loadArchive(loaded.manifest, data_path, error)) return nullptr;
    if (!impl->tuneGemms()) {
        if (error) *error = "GEMM algorithm selection failed";
        return nullptr;
    }
    return std::unique_ptr<HipTinyLlamaRunner>(new HipTinyLlamaRunner(std::move(impl)));
}

HipTinyLlamaRunner::HipTinyLlamaRunner(std::unique_ptr<Impl> impl) noexcept : impl_(std::move(impl)) {}
HipTinyLlamaRunner::~HipTinyLlamaRunner() = default;

TinyLlamaConfig HipTinyLlamaRunner::generationConfig() const noexcept { return impl_->cfg.model; }
std::uint32_t HipTinyLlamaRunner::generationMaxBatchSize() const noexcept { return impl_->cfg.max_positions; }
std::uint64_t HipTinyLlamaRunner::deviceWeightBytes() const noexcept { return impl_->weight_bytes; }
std::uint64_t HipTinyLlamaRunner::deviceWorkspaceBytes() const noexcept { return impl_->work_bytes; }

GenerationStepResult HipTinyLlamaRunner::generationForwardToken(RequestId request_id, std::uint32_t token_id,
                                                                std::uint32_t expected_position)
{
    GenerationBatchResult r = impl_->forward({GenerationSpan{request_id, expected_position, {token_id}}}, nullptr);
    if (!r.success) return GenerationStepResult{false, 0, std::move(r.detail)};
    return std::move(r.steps.front());
}

GenerationBatchResult HipTinyLlamaRunner::generationForwardBatch(std::vector<GenerationBatchItem> const& batch)
{
    std::vector<GenerationSpan> spans;
    spans.reserve(batch.size());
    for (GenerationBatchItem const& it : batch) spans.push_back({it.request_id, it.expected_position, {it.token_id}});
    return impl_->forward(spans, nullptr);
}

GenerationBatchResult HipTinyLlamaRunner::generationForwardSpans(std::vector<GenerationSpan> const& spans)
{
    return impl_->forward(spans, nullptr);
}

GenerationBatchResult HipTinyLlamaRunner::forwardSpans(std::vector<GenerationSpan> const& spans, float* host_logits)
{
    return impl_->forward(spans, host_logits);
}

void HipTinyLlamaRunner::watchLogits(std::vector<RequestId> ids, float* rows, std::uint32_t* positions,
                                     std::uint32_t* counts)
{
    bool const off = ids.empty() || rows == nullptr || positions == nullptr || counts == nullptr;
    impl_->watch_ids = off ? std::vector<RequestId>{} : std::move(ids);
    impl_->watch_rows = off ? nullptr : rows;
    impl_->watch_positions = off ? nullptr : positions;
    impl_->watch_counts = off ? nullptr : counts;
}

}  // namespace kimkvcache
