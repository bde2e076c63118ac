// attention_common.h -- MFMA operand types, LDS group tables and wave
// helpers shared by the paged decode and paged prefill kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.h"

namespace kimkv {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr unsigned kMaxChunk = 65536;     // tokens per chunk (multiple of 64)
constexpr unsigned kMaxGroups = kMaxChunk / 8;
constexpr float kLog2e = 1.4426950408889634f;

// One 8-token group of the chunk, 8 bytes so a 65536-token chunk's table
// fits in 64 KiB of LDS: `page` is the slot, with kExtentPage set for an
// extent page (kUnmappedGroup when no descriptor covers the group); `pt0` is
// the group's first token inside the page, `cap` the page's capacity.
constexpr uint32_t kExtentPage = 0x80000000u;
constexpr uint32_t kUnmappedGroup = 0xFFFFFFFFu;

struct GroupEntry {
    uint32_t page;
    uint16_t pt0;
    uint16_t cap;
};

// Resolves group entries to the (layer, head) block of their page for one
// (layer, KV head): block = page_base(slot) + head_block(layer, head), i.e.
// a per-kind base for this (layer, head) plus slot * slot_elements.
struct GroupResolver {
    const uint16_t* micro;
    const uint16_t* extent;
    uint64_t micro_slot_elements;
    uint64_t extent_slot_elements;

    __device__ GroupResolver(const PoolView& P, uint32_t layer, uint32_t head)
    {
        uint64_t const region = static_cast<uint64_t>(layer) * P.layer_elements;
        uint64_t const unit = static_cast<uint64_t>(head) * 2ull * P.dim;
        micro = P.micro + region + unit * P.micro_tokens;
        extent = P.extent + region + unit * P.extent_tokens;
        micro_slot_elements = P.micro_slot_elements;
        extent_slot_elements = P.extent_slot_elements;
    }

    __device__ const uint16_t* block(GroupEntry g) const
    {
        uint64_t const slot = g.page & ~kExtentPage;
        return (g.page & kExtentPage) != 0 ? extent + slot * extent_slot_elements
                                           : micro + slot * micro_slot_elements;
    }
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
__device__ inline void add_groups(const PoolView& P, kimkv_block_desc const& e, uint32_t c0, uint32_t c1,
                                  uint32_t T, GroupEntry* groups, uint32_t* s_generic)
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
    uint32_t const tag = e.kind == KIMKV_PAGE_EXTENT ? e.slot | kExtentPage : e.slot;
    for (uint32_t g = (lo - c0) >> 3; g < (hi - c0 + 7) >> 3; ++g) {
        groups[g] = GroupEntry{tag, static_cast<uint16_t>(c0 + 8 * g - b), static_cast<uint16_t>(cap)};
    }
}

}  // namespace kimkv
