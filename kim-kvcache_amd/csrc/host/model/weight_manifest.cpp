// Weight archive manifests: parsing, validation against the model config, and
// streamed SHA-256 of archive ranges.  Behaviour (accepted fields, tensor
// names and shapes, error codes and their precedence) follows the
// reference's src/model/weight_manifest.cpp:351-684, which its converter
// script and model runner rely on.  The digest is SHA-256 as FIPS 180-4
// defines it (the round constants and initial hash values below are the
// standard's).
#include "kim-kv/model/weight_manifest.h"

#include <algorithm>
#include <array>
#include <charconv>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <limits>
#include <map>
#include <set>
#include <utility>

namespace kimkvcache {
namespace {

constexpr std::uint32_t kSupportedVersion = 1;

WeightManifestStatus fail(WeightManifestError e, std::string detail)
{
    return WeightManifestStatus{e, std::move(detail)};
}

// ---- SHA-256 (FIPS 180-4) -------------------------------------------------------------------------

class Sha256 final {
public:
    void absorb(unsigned char const* data, std::size_t n) noexcept
    {
        length_ += n;
        if (fill_ != 0) {
            std::size_t const take = std::min(n, block_.size() - fill_);
            std::memcpy(block_.data() + fill_, data, take);
            fill_ += take;
            data += take;
            n -= take;
            if (fill_ < block_.size()) return;
            compress(block_.data());
            fill_ = 0;
        }
        for (; n >= 64; data += 64, n -= 64) compress(data);
        std::memcpy(block_.data(), data, n);
        fill_ = n;
    }

    std::string hex() noexcept
    {
        std::uint64_t const bits = length_ * 8;
        unsigned char pad[72] = {0x80};
        std::size_t const padding = (fill_ < 56 ? 56 : 120) - fill_;
        for (int i = 0; i < 8; ++i) pad[padding + i] = static_cast<unsigned char>(bits >> (56 - 8 * i));
        std::uint64_t const kept = length_;
        absorb(pad, padding + 8);
        length_ = kept;
        char text[65];
        for (int i = 0; i < 8; ++i) std::snprintf(text + 8 * i, 9, "%08x", h_[i]);
        return std::string(text, 64);
    }

private:
    static std::uint32_t rotr(std::uint32_t x, int n) noexcept { return (x >> n) | (x << (32 - n)); }

    void compress(unsigned char const* p) noexcept
    {
        static constexpr std::uint32_t k[64] = {
            0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
            0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
            0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
            0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
            0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
            0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
            0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
            0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2,
        };
        std::uint32_t w[64];
        for (int t = 0; t < 16; ++t) {
            w[t] = static_cast<std::uint32_t>(p[4 * t]) << 24 | static_cast<std::uint32_t>(p[4 * t + 1]) << 16
                | static_cast<std::uint32_t>(p[4 * t + 2]) << 8 | p[4 * t + 3];
        }
        for (int t = 16; t < 64; ++t) {
            std::uint32_t const s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
            std::uint32_t const s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
            w[t] = w[t - 16] + s0 + w[t - 7] + s1;
        }
        std::array<std::uint32_t, 8> v = h_;   // a b c d e f g h
        for (int t = 0; t < 64; ++t) {
            std::uint32_t const e = v[4];
            std::uint32_t const a = v[0];
            std::uint32_t const t1 = v[7] + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & v[5]) ^ (~e & v[6]))
                + k[t] + w[t];
            std::uint32_t const t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & v[1]) ^ (a & v[2]) ^ (v[1] & v[2]));
            std::move_backward(v.begin(), v.end() - 1, v.end());
            v[4] += t1;
            v[0] = t1 + t2;
        }
        for (int i = 0; i < 8; ++i) h_[i] += v[i];
    }

    std::array<std::uint32_t, 8> h_{0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                    0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    std::array<unsigned char, 64> block_{};
    std::size_t fill_{0};
    std::uint64_t length_{0};
};

// ---- field parsing -----------------------------------------------------------------------------------

bool toU64(std::string_view s, std::uint64_t& out) noexcept
{
    if (s.empty()) return false;
    auto const r = std::from_chars(s.data(), s.data() + s.size(), out);
    return r.ec == std::errc{} && r.ptr == s.data() + s.size();
}

bool toU32(std::string_view s, std::uint32_t& out) noexcept
{
    std::uint64_t v = 0;
    if (!toU64(s, v) || v > std::numeric_limits<std::uint32_t>::max()) return false;
    out = static_cast<std::uint32_t>(v);
    return true;
}

bool toF32(std::string const& s, float& out)
{
    if (s.empty()) return false;
    char* end = nullptr;
    float const v = std::strtof(s.c_str(), &end);
    if (end != s.c_str() + s.size()) return false;
    out = v;
    return true;
}

bool isDigest(std::string const& s) noexcept
{
    return s.size() == 64
        && std::all_of(s.begin(), s.end(), [](char c) { return (c >= '0' && c <= '9') || (c >= 'a' && c <= 'f'); });
}

std::vector<std::string_view> cut(std::string_view s, char sep)
{
    std::vector<std::string_view> parts;
    for (;;) {
        std::size_t const at = s.find(sep);
        parts.push_back(s.substr(0, at));
        if (at == std::string_view::npos) return parts;
        s.remove_prefix(at + 1);
    }
}

// Every scalar field of the format and where it goes; all are required.
using Setter = std::function<bool(std::string const&, WeightManifest&)>;

std::vector<std::pair<char const*, Setter>> const& fieldTable()
{
    auto text = [](std::string WeightManifest::*m) -> Setter {
        return [m](std::string const& v, WeightManifest& w) { return !v.empty() && (w.*m = v, true); };
    };
    auto u32 = [](std::uint32_t TinyLlamaConfig::*m) -> Setter {
        return [m](std::string const& v, WeightManifest& w) { return toU32(v, w.config.*m); };
    };
    auto f32 = [](float TinyLlamaConfig::*m) -> Setter {
        return [m](std::string const& v, WeightManifest& w) { return toF32(v, w.config.*m); };
    };
    static std::vector<std::pair<char const*, Setter>> const table = {
        {"version", [](std::string const& v, WeightManifest& w) { return toU32(v, w.version); }},
        {"checkpoint", text(&WeightManifest::checkpoint)},
        {"checkpoint_revision", text(&WeightManifest::checkpoint_revision)},
        {"tokenizer_revision", text(&WeightManifest::tokenizer_revision)},
        {"config_sha256", text(&WeightManifest::config_sha256)},
        {"dtype", text(&WeightManifest::data_type)},
        {"data_file", text(&WeightManifest::data_file)},
        {"data_bytes", [](std::string const& v, WeightManifest& w) { return toU64(v, w.data_bytes); }},
        {"hidden_size", u32(&TinyLlamaConfig::hidden_size)},
        {"intermediate_size", u32(&TinyLlamaConfig::intermediate_size)},
        {"layer_count", u32(&TinyLlamaConfig::layer_count)},
        {"attention_head_count", u32(&TinyLlamaConfig::attention_head_count)},
        {"kv_head_count", u32(&TinyLlamaConfig::kv_head_count)},
        {"head_dimension", u32(&TinyLlamaConfig::head_dimension)},
        {"vocabulary_size", u32(&TinyLlamaConfig::vocabulary_size)},
        {"max_position_embeddings", u32(&TinyLlamaConfig::max_position_embeddings)},
        {"bos_token_id", u32(&TinyLlamaConfig::bos_token_id)},
        {"eos_token_id", u32(&TinyLlamaConfig::eos_token_id)},
        {"rms_norm_epsilon", f32(&TinyLlamaConfig::rms_norm_epsilon)},
        {"rope_theta", f32(&TinyLlamaConfig::rope_theta)},
        {"tied_word_embeddings",
         [](std::string const& v, WeightManifest& w) {
             if (v != "0" && v != "1") return false;
             w.config.tied_word_embeddings = v == "1";
             return true;
         }},
    };
    return table;
}

// Tensor name -> shape for a config (Hugging Face Llama naming).
std::map<std::string, std::vector<std::uint32_t>> requiredTensors(TinyLlamaConfig const& c)
{
    std::uint32_t const H = c.hidden_size, I = c.intermediate_size, V = c.vocabulary_size;
    std::uint32_t const KV = c.kv_head_count * c.head_dimension;
    std::map<std::string, std::vector<std::uint32_t>> need = {
        {"model.embed_tokens.weight", {V, H}},
        {"model.norm.weight", {H}},
        {"lm_head.weight", {V, H}},
    };
    for (std::uint32_t l = 0; l < c.layer_count; ++l) {
        std::string const p = "model.layers." + std::to_string(l) + ".";
        need[p + "input_layernorm.weight"] = {H};
        need[p + "post_attention_layernorm.weight"] = {H};
        need[p + "self_attn.q_proj.weight"] = {H, H};
        need[p + "self_attn.k_proj.weight"] = {KV, H};
        need[p + "self_attn.v_proj.weight"] = {KV, H};
        need[p + "self_attn.o_proj.weight"] = {H, H};
        need[p + "mlp.gate_proj.weight"] = {I, H};
        need[p + "mlp.up_proj.weight"] = {I, H};
        need[p + "mlp.down_proj.weight"] = {H, I};
    }
    return need;
}

// fp16 elements of a 1-D or 2-D shape, false on a zero or overflowing size.
bool elementCount(std::vector<std::uint32_t> const& shape, std::uint64_t& n) noexcept
{
    if (shape.empty() || shape.size() > 2) return false;
    n = 1;
    for (std::uint32_t d : shape) {
        if (d == 0 || n > std::numeric_limits<std::uint64_t>::max() / 2 / d) return false;
        n *= d;
    }
    return true;
}

}  // namespace

WeightTensorDescriptor const* WeightManifest::find(std::string_view name) const noexcept
{
    for (WeightTensorDescriptor const& t : tensors) {
        if (t.name == name) return &t;
    }
    return nullptr;
}

WeightManifestStatus validateWeightManifest(WeightManifest const& m)
{
    if (m.version != kSupportedVersion) return fail(WeightManifestError::UnsupportedVersion, "manifest version must be 1");
    if (m.data_type != "fp16") return fail(WeightManifestError::UnsupportedDataType, "only fp16 archives are supported");
    if (!m.config.valid()) return fail(WeightManifestError::InvalidConfig, "model dimensions are inconsistent");
    if (m.checkpoint.empty() || m.checkpoint_revision.empty() || m.tokenizer_revision.empty()
        || !isDigest(m.config_sha256) || m.data_file.empty() || m.data_bytes == 0) {
        return fail(WeightManifestError::InvalidConfig, "model identity or data archive metadata is incomplete");
    }
    auto need = requiredTensors(m.config);
    std::set<std::string> seen;
    std::vector<std::pair<std::uint64_t, std::uint64_t>> spans;   // [begin, end) by tensor
    for (WeightTensorDescriptor const& t : m.tensors) {
        if (!seen.insert(t.name).second) return fail(WeightManifestError::DuplicateTensor, "duplicate tensor: " + t.name);
        auto const wanted = need.find(t.name);
        if (wanted == need.end()) return fail(WeightManifestError::UnexpectedTensor, "unexpected tensor: " + t.name);
        if (t.shape != wanted->second || !isDigest(t.sha256)) {
            return fail(WeightManifestError::InvalidTensor, "shape or checksum metadata mismatch: " + t.name);
        }
        std::uint64_t n = 0;
        if (!elementCount(t.shape, n) || t.offset % 2 != 0 || t.byte_size != 2 * n || t.offset > m.data_bytes
            || t.byte_size > m.data_bytes - t.offset) {
            return fail(WeightManifestError::InvalidTensor, "invalid byte range: " + t.name);
        }
        spans.emplace_back(t.offset, t.offset + t.byte_size);
        need.erase(wanted);
    }
    if (!need.empty()) return fail(WeightManifestError::MissingTensor, "missing tensor: " + need.begin()->first);
    std::vector<std::size_t> order(spans.size());
    for (std::size_t i = 0; i < order.size(); ++i) order[i] = i;
    std::sort(order.begin(), order.end(), [&spans](std::size_t a, std::size_t b) { return spans[a] < spans[b]; });
    for (std::size_t k = 1; k < order.size(); ++k) {
        if (spans[order[k]].first < spans[order[k - 1]].second) {
            return fail(WeightManifestError::InvalidTensor, "overlapping tensor ranges: " + m.tensors[order[k]].name);
        }
    }
    return {};
}

WeightManifestLoadResult loadWeightManifest(std::string const& manifest_path)
{
    WeightManifestLoadResult result;
    std::ifstream in(manifest_path);
    if (!in) {
        result.status = fail(WeightManifestError::FileOpenFailed, manifest_path);
        return result;
    }
    std::map<std::string, std::string> fields;
    std::vector<std::string> tensor_records;
    std::string line;
    for (std::size_t number = 1; std::getline(in, line); ++number) {
        if (line.empty() || line[0] == '#') continue;
        std::size_t const eq = line.find('=');
        if (eq == std::string::npos || eq == 0) {
            result.status = fail(WeightManifestError::ParseFailed, "invalid line " + std::to_string(number));
            return result;
        }
        std::string key = line.substr(0, eq);
        std::string value = line.substr(eq + 1);
        if (key == "tensor") {
            tensor_records.push_back(std::move(value));
        } else if (!fields.emplace(std::move(key), std::move(value)).second) {
            result.status = fail(WeightManifestError::ParseFailed, "duplicate key: " + line.substr(0, eq));
            return result;
        }
    }
    WeightManifest& m = result.manifest;
    bool complete = true;
    for (auto const& [key, set] : fieldTable()) {
        auto const it = fields.find(key);
        complete = complete && it != fields.end() && set(it->second, m);
    }
    std::uint32_t count = 0;
    auto const declared = fields.find("tensor_count");
    complete = complete && declared != fields.end() && toU32(declared->second, count);
    if (!complete || count != tensor_records.size()) {
        result.status = fail(WeightManifestError::ParseFailed, "missing field or tensor_count mismatch");
        return result;
    }
    m.tensors.reserve(tensor_records.size());
    for (std::string const& record : tensor_records) {
        std::vector<std::string_view> const f = cut(record, '|');
        if (f.size() != 5) {
            result.status = fail(WeightManifestError::ParseFailed, "tensor record must contain five fields");
            return result;
        }
        WeightTensorDescriptor t;
        t.name = std::string(f[0]);
        t.sha256 = std::string(f[4]);
        if (!toU64(f[1], t.offset) || !toU64(f[2], t.byte_size)) {
            result.status = fail(WeightManifestError::ParseFailed, "invalid tensor range: " + t.name);
            return result;
        }
        for (std::string_view d : cut(f[3], ',')) {
            std::uint32_t dim = 0;
            if (!toU32(d, dim)) {
                result.status = fail(WeightManifestError::ParseFailed, "invalid tensor shape: " + t.name);
                return result;
            }
            t.shape.push_back(dim);
        }
        m.tensors.push_back(std::move(t));
    }
    result.status = validateWeightManifest(m);
    return result;
}

WeightManifestStatus computeWeightDataSha256(std::string const& data_path, std::uint64_t offset,
                                             std::uint64_t byte_size, std::string& sha256)
{
    sha256.clear();
    if (data_path.empty() || byte_size == 0
        || offset > static_cast<std::uint64_t>(std::numeric_limits<std::streamoff>::max())) {
        return fail(WeightManifestError::InvalidArgument, "invalid checksum range");
    }
    std::ifstream in(data_path, std::ios::binary);
    if (!in) return fail(WeightManifestError::FileOpenFailed, data_path);
    in.seekg(static_cast<std::streamoff>(offset));
    std::vector<unsigned char> piece(std::size_t{1} << 22);
    Sha256 digest;
    for (std::uint64_t left = byte_size; left != 0;) {
        auto const want = static_cast<std::size_t>(std::min<std::uint64_t>(left, piece.size()));
        in.read(reinterpret_cast<char*>(piece.data()), static_cast<std::streamsize>(want));
        if (in.gcount() != static_cast<std::streamsize>(want)) {
            return fail(WeightManifestError::DataFileMismatch, "checksum range exceeds data file");
        }
        digest.absorb(piece.data(), want);
        left -= want;
    }
    sha256 = digest.hex();
    return {};
}

WeightManifestStatus validateWeightDataFile(WeightManifest const& m, std::string const& data_path)
{
    WeightManifestStatus const meta = validateWeightManifest(m);
    if (!meta.ok()) return meta;
    std::ifstream in(data_path, std::ios::binary | std::ios::ate);
    if (!in) return fail(WeightManifestError::FileOpenFailed, data_path);
    std::streamoff const size = in.tellg();
    if (size < 0 || static_cast<std::uint64_t>(size) != m.data_bytes) {
        return fail(WeightManifestError::DataFileMismatch, "archive size differs from manifest");
    }
    for (WeightTensorDescriptor const& t : m.tensors) {
        std::string actual;
        WeightManifestStatus const s = computeWeightDataSha256(data_path, t.offset, t.byte_size, actual);
        if (!s.ok()) return s;
        if (actual != t.sha256) return fail(WeightManifestError::ChecksumMismatch, t.name);
    }
    return {};
}

}  // namespace kimkvcache
