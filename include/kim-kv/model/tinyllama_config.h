#pragma once

// Llama-family shape contract of the generation runtime and the model runner
// (include/kim-kv/model/tinyllama_config.h:1-60 of the reference; same field
// order so aggregate initialisers written against the reference compile).

#include <cstdint>

namespace kimkvcache {

struct TinyLlamaConfig final {
    std::uint32_t hidden_size{0};
    std::uint32_t intermediate_size{0};
    std::uint32_t layer_count{0};
    std::uint32_t attention_head_count{0};
    std::uint32_t kv_head_count{0};
    std::uint32_t head_dimension{0};
    std::uint32_t vocabulary_size{0};
    std::uint32_t max_position_embeddings{0};
    std::uint32_t bos_token_id{0};
    std::uint32_t eos_token_id{0};
    float rms_norm_epsilon{0.0F};
    float rope_theta{0.0F};
    bool tied_word_embeddings{false};

    // Heads tile the hidden size, query heads group evenly over KV heads,
    // RoPE needs an even head dimension, special tokens are in the vocabulary.
    [[nodiscard]] constexpr bool valid() const noexcept
    {
        return hidden_size != 0 && intermediate_size != 0 && layer_count != 0 && attention_head_count != 0
            && kv_head_count != 0 && head_dimension != 0 && hidden_size == attention_head_count * head_dimension
            && attention_head_count >= kv_head_count && attention_head_count % kv_head_count == 0
            && head_dimension % 2 == 0 && vocabulary_size != 0 && max_position_embeddings != 0
            && bos_token_id < vocabulary_size && eos_token_id < vocabulary_size && rms_norm_epsilon > 0.0F
            && rope_theta > 0.0F;
    }
};

// TinyLlama 1.1B Chat: 22 layers, hidden 2048, SwiGLU 5632, 32 q / 4 kv heads
// x 64, vocabulary 32000, 2048 positions, RMSNorm eps 1e-5, RoPE theta 1e4.
[[nodiscard]] constexpr TinyLlamaConfig tinyLlama11bChatConfig() noexcept
{
    return TinyLlamaConfig{2048, 5632, 22, 32, 4, 64, 32000, 2048, 1, 2, 1.0e-5F, 10000.0F, false};
}

}  // namespace kimkvcache
