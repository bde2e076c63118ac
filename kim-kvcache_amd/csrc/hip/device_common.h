// device_common.h -- shared device-side definitions for the gfx950 KV kernels.
//
// Page layout (see include/kimkv_hip.h): per (layer, head) a contiguous block
// of 2*cap*D halves, K first, then V transposed, both cut into 32-wide blocks
// (k_offset / v_offset below).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <atomic>
#include <cstdint>
#include <mutex>

#include "kimkv_hip.h"

// Work-counter slots of persistent launches: each stream that makes such a
// launch on a storage owns one slot for the storage's lifetime, and a
// launch's last workgroup resets its slot.  Launches on one stream run in
// order, so the next launch on that stream finds the slot cleared, and
// launches on different streams never share a slot.
constexpr uint32_t kWorkCounterSlots = 64;
constexpr uint32_t kWorkCounterStride = 64;   // words: one slot per 256-byte line

struct kimkv_storage {
    kimkv_layout layout{};
    uint32_t micro_capacity{0};
    uint32_t extent_capacity{0};
    uint16_t micro_tokens{0};
    uint16_t extent_tokens{0};
    uint64_t micro_page_elements{0};   // one page, every layer
    uint64_t extent_page_elements{0};
    uint16_t* pool{nullptr};           // the one allocation (layer-major, see page_base)
    uint16_t* micro{nullptr};          // layer 0's micro blocks
    uint16_t* extent{nullptr};         // layer 0's extent blocks
    uint32_t* faults{nullptr};        // device word, KIMKV_FAULT_* bits
    uint32_t* work_counters{nullptr}; // kWorkCounterSlots slots of kWorkCounterStride words
    mutable std::mutex work_counter_mutex;
    mutable void* work_counter_stream[kWorkCounterSlots]{};   // slot owners
    mutable uint32_t work_counter_owners{0};
    uint32_t* fault_host{nullptr};    // mapped pinned word kimkv_storage_faults reads
    uint32_t* fault_view{nullptr};    // its device address
    int device{0};
    int compute_units{0};
};

namespace kimkv {

constexpr unsigned kWave = 64;

// Pool view passed to kernels by value.
struct PoolView {
    uint16_t* micro;
    uint16_t* extent;
    uint64_t micro_slot_elements;    // one micro page's block of one layer (every head)
    uint64_t extent_slot_elements;
    uint64_t layer_elements;         // one layer's region: every micro, then every extent page
    uint32_t micro_capacity;
    uint32_t extent_capacity;
    uint32_t micro_tokens;
    uint32_t extent_tokens;
    uint32_t layers;
    uint32_t heads;
    uint32_t dim;
    uint32_t* faults;
};

// Elements of one page's block of one layer (K and V^T of every head).
inline uint64_t slot_elements(const kimkv_layout& l, uint32_t page_tokens)
{
    return 2ull * l.kv_heads * l.head_dim * page_tokens;
}

inline PoolView pool_view(const kimkv_storage& s)
{
    uint64_t const micro_slot = slot_elements(s.layout, s.micro_tokens);
    uint64_t const extent_slot = slot_elements(s.layout, s.extent_tokens);
    return PoolView{s.micro, s.extent, micro_slot, extent_slot,
                    micro_slot * s.micro_capacity + extent_slot * s.extent_capacity,
                    s.micro_capacity, s.extent_capacity, s.micro_tokens, s.extent_tokens,
                    s.layout.layers, s.layout.kv_heads, s.layout.head_dim, s.faults};
}

// A workgroup that skips its job or item because the job or item is invalid
// records why in the storage's fault word (read and cleared by
// kimkv_storage_faults).  Called with a workgroup-uniform condition; one
// thread writes, with a device-scope atomic.
__device__ inline void report_fault(const PoolView& p, uint32_t bit)
{
    if (threadIdx.x == 0 && p.faults != nullptr) atomicOr(p.faults, bit);
}

// The pools are one allocation, layer-major: `layers` regions of
// layer_elements each; region l holds every micro page's layer-l block, then
// every extent page's, and a page's block holds its heads one after the
// other.  So the (layer, head) block of a page is
//   pool + l * layer_elements + [micro part] + slot * slot_elements(kind)
//        + head * 2 * cap * D,
// page_base() being the layer-0 block and head_block() the rest.  A decode
// or prefill launch works on one layer, and one layer's blocks of all pages
// lie in one region (8.6 GB for 131 072 extent pages of 4 heads x 64 dims)
// instead of being spread over the whole pool: random 16 KiB pieces stream
// at 7.0 TB/s from one region against 6.7 TB/s from a 189 GB span
// (measured on MI355X; the difference is address-translation reach).
//
// Layer-0 block of a (kind, slot), or nullptr when the handle does not name
// a page of this storage or its declared capacity disagrees with the pool's.
__device__ inline uint16_t* page_base(const PoolView& p, uint32_t kind, uint32_t slot,
                                      uint32_t capacity)
{
    if (kind == KIMKV_PAGE_MICRO) {
        if (slot >= p.micro_capacity || capacity != p.micro_tokens || p.micro == nullptr) {
            return nullptr;
        }
        return p.micro + static_cast<uint64_t>(slot) * p.micro_slot_elements;
    }
    if (kind == KIMKV_PAGE_EXTENT) {
        if (slot >= p.extent_capacity || capacity != p.extent_tokens || p.extent == nullptr) {
            return nullptr;
        }
        return p.extent + static_cast<uint64_t>(slot) * p.extent_slot_elements;
    }
    return nullptr;
}

__device__ inline uint32_t pool_tokens(const PoolView& p, uint32_t kind)
{
    return kind == KIMKV_PAGE_MICRO ? p.micro_tokens : p.extent_tokens;
}

// Element offset of a page's (layer, head) block from its page_base(), for
// a page of `cap` tokens.
__device__ inline uint64_t head_block(const PoolView& p, uint32_t cap, uint32_t layer, uint32_t head)
{
    return static_cast<uint64_t>(layer) * p.layer_elements + static_cast<uint64_t>(head) * 2ull * cap * p.dim;
}

// Inside a (layer, head) block of a page with `cap` tokens and head dim D:
//   K(t, d) = (d / kw) * cap * kw + t * kw + d % kw,             kw = k_width(D)
//   V(t, d) = cap * D + (t / vw) * D * vw + d * vw + t % vw,      vw = v_width(cap)
// K is split into 32-dim column blocks and V^T into 32-token column blocks,
// so the 16-byte loads of one decode instruction (16 tokens x 8 dims of K,
// or 16 dims x 8 tokens of V) land on whole 64-byte row pieces that tile
// complete 128-byte lines.  8 consecutive dims of K (d % 8 == 0) and 8
// consecutive tokens of V (t % 8 == 0) stay contiguous whenever D and cap
// are multiples of 8.
__host__ __device__ inline uint32_t k_width(uint32_t D) { return D % 32u == 0u ? 32u : D; }
__host__ __device__ inline uint32_t v_width(uint32_t cap) { return cap % 32u == 0u ? 32u : cap; }

__host__ __device__ inline uint64_t k_offset(uint32_t cap, uint32_t D, uint32_t t, uint32_t d)
{
    uint32_t const kw = k_width(D);
    return static_cast<uint64_t>(d / kw) * cap * kw + static_cast<uint64_t>(t) * kw + d % kw;
}

__host__ __device__ inline uint64_t v_offset(uint32_t cap, uint32_t D, uint32_t t, uint32_t d)
{
    uint32_t const vw = v_width(cap);
    return static_cast<uint64_t>(cap) * D + static_cast<uint64_t>(t / vw) * D * vw + static_cast<uint64_t>(d) * vw
        + t % vw;
}

// ---- XCD-aware workgroup order ----------------------------------------------
// MI355X dispatches the workgroups of a launch round-robin over its 8 XCDs
// (workgroup w runs on XCD w % 8), each with its own L2.  This maps dispatch
// index w of an n-workgroup grid to a logical index such that XCD x receives
// one contiguous logical range (the first n % 8 XCDs one element longer), so
// workgroups that read the same data share an L2.  A bijection on [0, n).
constexpr unsigned kXcds = 8;
__host__ __device__ inline uint32_t xcd_logical_index(uint32_t w, uint32_t n)
{
    uint32_t const per = (n + kXcds - 1) / kXcds;
    uint32_t const tall = n % kXcds == 0 ? kXcds : n % kXcds;
    uint32_t const x = w % kXcds;
    uint32_t const local = w / kXcds;
    return x < tall ? x * per + local : tall * per + (x - tall) * (per - 1) + local;
}

// ---- synthetic generator (bit-identical to kimkv_synth_value) -------------
__host__ __device__ inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__host__ __device__ inline int32_t synth_int(uint64_t seed, uint64_t row, uint32_t col)
{
    uint64_t const h = mix64(mix64(seed + row * 0x9E3779B97F4A7C15ull) + col);
    return static_cast<int32_t>(h & 0xFFFFu) + static_cast<int32_t>((h >> 16) & 0xFFFFu)
        + static_cast<int32_t>((h >> 32) & 0xFFFFu) + static_cast<int32_t>(h >> 48) - 131070;
}

__device__ inline uint16_t synth_f16(uint64_t seed, uint64_t row, uint32_t col)
{
    float const x = static_cast<float>(synth_int(seed, row, col)) * (1.0f / 32768.0f);
    return __half_as_ushort(__float2half_rn(x));
}

__host__ __device__ inline uint64_t kv_row(uint32_t stream, uint32_t layer, uint32_t component,
                                           uint32_t token)
{
    return (static_cast<uint64_t>(stream & 0xFFFFu) << 48)
        | (static_cast<uint64_t>(layer & 0x7FFFu) << 33)
        | (static_cast<uint64_t>(component & 1u) << 32) | static_cast<uint64_t>(token);
}

// ---- wave-parallel page-table search ----------------------------------------
// Index of the last descriptor whose logical_token_begin <= token (descriptors
// are sorted by begin).  64-ary search: each round every lane probes one
// candidate, so a 4096-entry table resolves in two dependent rounds.
// Must be called by all 64 lanes of a wave; the result is wave-uniform.
__device__ inline uint32_t find_descriptor_wave(const kimkv_block_desc* d, uint32_t count,
                                                uint32_t token)
{
    uint32_t const lane = threadIdx.x & (kWave - 1);
    uint32_t lo = 0;
    uint32_t hi = count;
    while (hi - lo > 1) {
        uint32_t const step = (hi - lo + kWave - 1) / kWave;
        uint32_t const i = lo + lane * step;
        bool const pred = i < hi && d[i].logical_token_begin <= token;
        uint64_t const mask = __ballot(pred);
        if (mask == 0) {
            return lo;
        }
        uint32_t const last = 63u - static_cast<uint32_t>(__clzll(mask));
        lo = lo + last * step;
        hi = min(lo + step, hi);
    }
    return lo;
}

inline uint32_t ceil_div(uint64_t a, uint64_t b) { return static_cast<uint32_t>((a + b - 1) / b); }

}  // namespace kimkv
