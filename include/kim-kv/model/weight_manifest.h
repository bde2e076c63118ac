// Weight archive manifest of a TinyLlama-shaped checkpoint (the reference's
// include/kim-kv/model/weight_manifest.h:1-136; same types, names and error
// codes).  A manifest is a text file of `key=value` lines (blank lines and
// lines starting with '#' ignored): model identity (version, checkpoint,
// checkpoint_revision, tokenizer_revision, config_sha256, dtype, data_file,
// data_bytes), the model dimensions of TinyLlamaConfig, tensor_count, and one
// `tensor=name|offset|byte_size|d0[,d1]|sha256` line per tensor of the fp16
// data file.  Tensor names are the Hugging Face Llama ones
// (model.embed_tokens.weight, model.layers.<l>.self_attn.q_proj.weight, ...).
#pragma once

#include "kim-kv/model/tinyllama_config.h"

#include <cstdint>
#include <string>
#include <string_view>
#include <vector>

namespace kimkvcache {

enum class WeightManifestError : std::uint8_t {
    None,
    InvalidArgument,
    FileOpenFailed,
    ParseFailed,
    UnsupportedVersion,
    UnsupportedDataType,
    InvalidConfig,
    InvalidTensor,
    DuplicateTensor,
    MissingTensor,
    UnexpectedTensor,
    DataFileMismatch,
    ChecksumMismatch,
};

[[nodiscard]] constexpr std::string_view toString(WeightManifestError error) noexcept
{
    switch (error) {
    case WeightManifestError::None: return "none";
    case WeightManifestError::InvalidArgument: return "invalid_argument";
    case WeightManifestError::FileOpenFailed: return "file_open_failed";
    case WeightManifestError::ParseFailed: return "parse_failed";
    case WeightManifestError::UnsupportedVersion: return "unsupported_version";
    case WeightManifestError::UnsupportedDataType: return "unsupported_data_type";
    case WeightManifestError::InvalidConfig: return "invalid_config";
    case WeightManifestError::InvalidTensor: return "invalid_tensor";
    case WeightManifestError::DuplicateTensor: return "duplicate_tensor";
    case WeightManifestError::MissingTensor: return "missing_tensor";
    case WeightManifestError::UnexpectedTensor: return "unexpected_tensor";
    case WeightManifestError::DataFileMismatch: return "data_file_mismatch";
    case WeightManifestError::ChecksumMismatch: return "checksum_mismatch";
    }
    return "unknown";
}

struct WeightManifestStatus final {
    WeightManifestError error{WeightManifestError::None};
    std::string detail{};

    [[nodiscard]] bool ok() const noexcept { return error == WeightManifestError::None; }
    [[nodiscard]] explicit operator bool() const noexcept { return ok(); }
};

struct WeightTensorDescriptor final {
    std::string name{};
    std::uint64_t offset{0};
    std::uint64_t byte_size{0};
    std::vector<std::uint32_t> shape{};
    std::string sha256{};   // 64 lowercase hex digits
};

struct WeightManifest final {
    std::uint32_t version{0};
    std::string checkpoint{};
    std::string checkpoint_revision{};
    std::string tokenizer_revision{};
    std::string config_sha256{};
    std::string data_type{};
    std::string data_file{};
    std::uint64_t data_bytes{0};
    TinyLlamaConfig config{};
    std::vector<WeightTensorDescriptor> tensors{};

    [[nodiscard]] WeightTensorDescriptor const* find(std::string_view name) const noexcept;
};

struct WeightManifestLoadResult final {
    WeightManifestStatus status{};
    WeightManifest manifest{};

    [[nodiscard]] bool ok() const noexcept { return status.ok(); }
};

// Parses and validates a manifest file.
[[nodiscard]] WeightManifestLoadResult loadWeightManifest(std::string const& manifest_path);

// Version 1, fp16, a valid model config, complete identity metadata, and
// exactly the tensors the config implies, each with its shape, an fp16 byte
// size, an in-range byte range and a well-formed digest; ranges may not
// overlap.
[[nodiscard]] WeightManifestStatus validateWeightManifest(WeightManifest const& manifest);

// The data file has exactly data_bytes bytes and every tensor range hashes to
// its SHA-256 (read in bounded pieces, never the whole archive at once).
[[nodiscard]] WeightManifestStatus validateWeightDataFile(WeightManifest const& manifest,
                                                          std::string const& data_path);

// SHA-256 (lowercase hex) of bytes [offset, offset + byte_size) of a file,
// streamed.
[[nodiscard]] WeightManifestStatus computeWeightDataSha256(std::string const& data_path, std::uint64_t offset,
                                                           std::uint64_t byte_size, std::string& sha256);

}  // namespace kimkvcache
