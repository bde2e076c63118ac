// attention_common.h -- MFMA operand types, LDS group tables and wave
// helpers shared by the paged decode and paged prefill kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.h"

namespace kimkv {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr unsigned kMaxChunk = 16384;     // tokens per chunk (multiple of 64)
constexpr unsigned kMaxGroups = kMaxChunk / 8;
constexpr float kLog2e = 1.4426950408889634f;

// One 8-token group of the chunk: `base` is the page's (layer, head 0) block.
struct GroupEntry {
    const uint16_t* base;
    uint32_t cap;
    uint32_t pt0;
};

__device__ inline float wave_max(float v)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}

__device__ inline float wave_sum(float v)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

__device__ inline half8_t load_half8(const uint16_t* p)
{
    return *reinterpret_cast<const half8_t*>(p);
}

// K/V page rows are read once per launch: non-temporal loads stream them
// without displacing reusable lines (measured on MI355X: a plain 16-byte
// streaming read reaches ~6.2 TB/s, the non-temporal form ~6.9 TB/s).
//
// The page pointers come out of the LDS group table as generic pointers; the
// address-space cast makes these global (not flat) loads, which count only
// against vmcnt, so waiting for a later LDS read does not also wait for the
// K/V bytes in flight.
typedef const __attribute__((address_space(1))) half8_t global_half8_t;

__device__ inline half8_t load_half8_stream(const uint16_t* p)
{
    return __builtin_nontemporal_load((global_half8_t*)(p));
}

// Records the 8-token groups of [c0, c1) that entry `e` covers.  An entry
// whose pages do not keep 8-token groups aligned (or names no page of the
// storage) switches the chunk to the generic path.
__device__ inline void add_groups(const PoolView& P, kimkv_block_desc const& e, uint32_t layer, uint32_t c0,
                                  uint32_t c1, uint32_t T, GroupEntry* groups, uint32_t* s_generic)
{
    uint32_t const b = e.logical_token_begin;
    uint32_t const end = b + e.valid_tokens;
    uint32_t const lo = max(b, c0);
    uint32_t const hi = min(end, c1);
    if (lo >= hi) return;
    uint32_t const cap = e.page_token_capacity;
    const uint16_t* page = page_base(P, e.kind, e.slot, cap);
    bool const aligned = (b & 7u) == 0 && (cap & 7u) == 0 && e.valid_tokens <= cap
        && ((end & 7u) == 0 || end >= T) && page != nullptr;
    if (!aligned) {
        *s_generic = 1;
        return;
    }
    const uint16_t* base = page + head_block(P, cap, layer, 0);
    for (uint32_t g = (lo - c0) >> 3; g < (hi - c0 + 7) >> 3; ++g) {
        groups[g] = GroupEntry{base, cap, c0 + 8 * g - b};
    }
}

}  // namespace kimkv
