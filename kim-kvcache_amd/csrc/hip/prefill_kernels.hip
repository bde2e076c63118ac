// prefill_kernels.hip -- multi-token causal GQA paged attention (chunked
// prefill) for gfx950.
//
// The reference has no such kernel: a prompt chunk advances one position at a
// time through single-token transactions (src/engine/iteration_scheduler.cpp:
// 545-657 driving paged_decode_kernels.cu:132-298), so prompt token i of a
// chunk attends to the first T0 + i + 1 tokens of the table.  This kernel
// computes the same outputs for all n positions of a chunk in one launch: new
// token i (0 <= i < n, position T - n + i of a table of T tokens whose last n
// tokens are the chunk) attends keys [0, T - n + i] of its KV head.
//
// Work: block = (item, KV head, block of 4*tpw new tokens), one wave per tpw
// tokens, where a wave's 16 MFMA columns are tpw tokens x G query heads
// (tpw = 16 / G).  Each wave streams the keys up to its last token's position
// in 64-token steps: S^T = K.Q^T and O^T += V^T.P^T on
// v_mfma_f32_16x16x32_f16 (same operand layout as the decode kernel), online
// softmax in base 2, fp32 accumulation, fp16 output.  Keys past a column's
// causal limit are masked per column.  The group table (8-token groups of the
// key range) is built in LDS one 8192-token segment at a time.  Tables that
// do not keep 8-token groups aligned, head dims other than 64 and group sizes
// that do not divide 16 take a one-row-at-a-time generic path.
#include <hip/hip_runtime.h>

#include <cmath>

#include "attention_common.h"
#include "device_common.h"
#include "runtime_internal.h"

namespace kimkv {
namespace {

constexpr unsigned kBlock = 256;   // 4 waves

struct PrefillShape {
    uint32_t tpw;        // new tokens per wave
    uint32_t G;          // query heads per KV head
    bool mfma;           // D == 64 and G divides 16
};

__device__ inline PrefillShape prefill_shape(uint32_t QH, uint32_t H, uint32_t D)
{
    uint32_t const G = QH / H;
    bool const mfma = D == 64 && G >= 1 && G <= 16 && 16 % G == 0;
    return PrefillShape{mfma ? 16 / G : 1, G, mfma};
}

// One wave, fast path: new tokens [i0, i0 + tpw) x the G query heads of KV
// head h; keys [s0, s1) of the current segment, whose groups are in `groups`
// (group g covers keys s0 + 8g ..).
struct PrefillWave {
    uint32_t l, a, r, x;
    bool qvalid;
    uint32_t limit;          // last key this lane's column may see
    uint64_t head_unit;
    half8_t qb0, qb1;
    float scale2;
    float m_run, l_part;
    float4_t acc[4];
};

__device__ void prefill_wave_init(PrefillWave& w, const kimkv_prefill_item& item, uint32_t h, uint32_t G, uint32_t QH,
                                  uint32_t i0)
{
    constexpr uint32_t D = 64;
    w.l = threadIdx.x & 63u;
    w.a = w.l >> 4;
    w.r = w.l & 15u;
    w.x = (w.l >> 2) & 3u;
    uint32_t const i = i0 + w.r / G;                     // new-token index of this lane's column
    uint32_t const q = h * G + w.r % G;
    w.qvalid = i < item.new_tokens;
    w.limit = item.token_count - item.new_tokens + (w.qvalid ? i : 0);
    w.head_unit = static_cast<uint64_t>(h) * 2u * D;
    half8_t const zero8 = {};
    w.qb0 = zero8;
    w.qb1 = zero8;
    if (w.qvalid) {
        const uint16_t* qrow = item.query + (static_cast<uint64_t>(i) * QH + q) * D;
        w.qb0 = *reinterpret_cast<const half8_t*>(qrow + w.a * 8);
        w.qb1 = *reinterpret_cast<const half8_t*>(qrow + 32 + w.a * 8);
    }
    w.scale2 = item.attention_scale * kLog2e;
    w.m_run = -INFINITY;
    w.l_part = 0.0f;
#pragma unroll
    for (uint32_t db = 0; db < 4; ++db) w.acc[db] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
}

// Keys [t0, t0 + 64) of the segment starting at s0 (ending at s1).
__device__ void prefill_wave_step(PrefillWave& w, const GroupEntry* groups, uint32_t s0, uint32_t s1, uint32_t t0)
{
    constexpr uint32_t D = 64;
    half8_t const zero8 = {};
    uint32_t const tg = (t0 - s0) >> 3;
    uint32_t const nvalid = s1 - t0;
    half8_t kop[2][2][2];
    half8_t vop[2][4];
#pragma unroll
    for (uint32_t kb = 0; kb < 2; ++kb) {
        GroupEntry const gk = groups[tg + 4 * kb + w.x];
#pragma unroll
        for (uint32_t e = 0; e < 2; ++e) {
            uint32_t const tt = 32 * kb + 8 * w.x + 4 * e + (w.l & 3u);
            if (tt < nvalid && gk.base != nullptr) {
                const uint16_t* row = gk.base + gk.cap * w.head_unit
                    + static_cast<uint64_t>(gk.pt0 + 4 * e + (w.l & 3u)) * 32 + w.a * 8;
                kop[kb][e][0] = load_half8_stream(row);
                kop[kb][e][1] = load_half8_stream(row + static_cast<uint64_t>(gk.cap) * 32);
            } else {
                kop[kb][e][0] = zero8;
                kop[kb][e][1] = zero8;
            }
        }
        GroupEntry const gv = groups[tg + 4 * kb + w.a];
        uint32_t const vt0 = 32 * kb + 8 * w.a;
        if (vt0 < nvalid && gv.base != nullptr) {
            uint32_t const vw = v_width(gv.cap);
            const uint16_t* vt = gv.base + gv.cap * w.head_unit + v_offset(gv.cap, D, gv.pt0, w.r);
#pragma unroll
            for (uint32_t db = 0; db < 4; ++db) vop[kb][db] = load_half8_stream(vt + static_cast<uint64_t>(db * 16) * vw);
            if (vt0 + 8 > nvalid) {
                uint32_t const keep = nvalid - vt0;
#pragma unroll
                for (uint32_t db = 0; db < 4; ++db) {
#pragma unroll
                    for (uint32_t j = 0; j < 8; ++j) {
                        if (j >= keep) vop[kb][db][j] = static_cast<_Float16>(0.0f);
                    }
                }
            }
        } else {
#pragma unroll
            for (uint32_t db = 0; db < 4; ++db) vop[kb][db] = zero8;
        }
    }

    float4_t s[2][2];
#pragma unroll
    for (uint32_t kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (uint32_t e = 0; e < 2; ++e) {
            float4_t z = {};
            z = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[kb][e][0], w.qb0, z, 0, 0, 0);
            s[kb][e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[kb][e][1], w.qb1, z, 0, 0, 0);
        }
    }
    // Element i of s[kb][e] is key t0 + 32kb + 8a + 4e + i for this lane's column.
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (uint32_t e = 0; e < 2; ++e) {
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) {
                uint32_t const tt = 32 * kb + 8 * w.a + 4 * e + i;
                bool const ok = tt < nvalid && t0 + tt <= w.limit;
                float const v = ok ? s[kb][e][i] * w.scale2 : -INFINITY;
                s[kb][e][i] = v;
                mx = fmaxf(mx, v);
            }
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    float const m_new = fmaxf(w.m_run, mx);
    // A column whose keys in this step are all masked keeps its state.
    float const alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(w.m_run - m_new);
    w.m_run = m_new;
    half8_t pb[2];
    float psum = 0.0f;
#pragma unroll
    for (uint32_t kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (uint32_t e = 0; e < 2; ++e) {
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) {
                float const p = m_new == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[kb][e][i] - m_new);
                psum += p;
                pb[kb][4 * e + i] = static_cast<_Float16>(p);
            }
        }
    }
    w.l_part = w.l_part * alpha + psum;
#pragma unroll
    for (uint32_t db = 0; db < 4; ++db) w.acc[db] *= alpha;
#pragma unroll
    for (uint32_t kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (uint32_t db = 0; db < 4; ++db) {
            w.acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop[kb][db], pb[kb], w.acc[db], 0, 0, 0);
        }
    }
}

__device__ void prefill_wave_store(PrefillWave& w, const kimkv_prefill_item& item, uint32_t h, uint32_t G,
                                   uint32_t QH, uint32_t i0)
{
    constexpr uint32_t D = 64;
    float l_tot = w.l_part + __shfl_xor(w.l_part, 16);
    l_tot += __shfl_xor(l_tot, 32);
    if (!w.qvalid) return;
    uint32_t const i = i0 + w.r / G;
    uint32_t const q = h * G + w.r % G;
    float const inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    uint16_t* out = item.output + (static_cast<uint64_t>(i) * QH + q) * D;
#pragma unroll
    for (uint32_t db = 0; db < 4; ++db) {
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) {
            out[db * 16 + 4 * w.a + k] = __half_as_ushort(__float2half_rn(w.acc[db][k] * inv));
        }
    }
}

// Generic path: one (new token, query head) row at a time; lanes own keys for
// the scores and dims for the output.
struct GenericScratch {
    float p[64];
    const uint16_t* head[64];
    uint32_t cap[64];
    uint32_t pt[64];
};

__device__ void prefill_row_generic(const PoolView& P, const kimkv_prefill_item& item, uint32_t h, uint32_t q,
                                    uint32_t i, uint32_t QH, GenericScratch* scratch)
{
    uint32_t const lane = threadIdx.x & 63u;
    uint32_t const D = P.dim;
    uint32_t const layer = item.layer;
    uint32_t const limit = item.token_count - item.new_tokens + i;   // inclusive
    float const scale2 = item.attention_scale * kLog2e;
    const uint16_t* qv = item.query + (static_cast<uint64_t>(i) * QH + q) * D;
    float m_run = -INFINITY;
    float l_run = 0.0f;
    float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t t0 = 0; t0 <= limit; t0 += 64) {
        uint32_t const t = t0 + lane;
        uint32_t idx = find_descriptor_wave(item.descriptors, item.descriptor_count, t0);
        const uint16_t* hb = nullptr;
        uint32_t cap = 0;
        uint32_t pt = 0;
        if (t <= limit) {
            while (idx + 1 < item.descriptor_count && item.descriptors[idx + 1].logical_token_begin <= t) ++idx;
            kimkv_block_desc const e = item.descriptors[idx];
            if (t >= e.logical_token_begin && t < e.logical_token_begin + e.valid_tokens
                && e.valid_tokens <= e.page_token_capacity) {
                const uint16_t* page = page_base(P, e.kind, e.slot, e.page_token_capacity);
                if (page != nullptr) {
                    cap = e.page_token_capacity;
                    pt = t - e.logical_token_begin;
                    hb = page + head_block(P, cap, layer, h);
                }
            }
        }
        float s = -INFINITY;
        if (hb != nullptr) {
            float dot = 0.0f;
            for (uint32_t d = 0; d < D; ++d) {
                dot += __half2float(__ushort_as_half(qv[d])) * __half2float(__ushort_as_half(hb[k_offset(cap, D, pt, d)]));
            }
            s = dot * scale2;
        }
        float const m_new = fmaxf(m_run, wave_max(s));
        float const alpha = m_new == -INFINITY ? 1.0f : exp2f(m_run - m_new);
        float const p = (hb != nullptr && m_new != -INFINITY) ? exp2f(s - m_new) : 0.0f;
        l_run = l_run * alpha + wave_sum(p);
        m_run = m_new;
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] *= alpha;
        scratch->p[lane] = p;
        scratch->head[lane] = hb;
        scratch->cap[lane] = cap;
        scratch->pt[lane] = pt;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        uint32_t const nt = min(64u, limit + 1 - t0);
        for (uint32_t tt = 0; tt < nt; ++tt) {
            float const pp = scratch->p[tt];
            const uint16_t* vb = scratch->head[tt];
            if (vb == nullptr || pp == 0.0f) continue;
            uint32_t const vc = scratch->cap[tt];
            uint32_t const vp = scratch->pt[tt];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint32_t const d = lane + 64u * k;
                if (d < D) o[k] += pp * __half2float(__ushort_as_half(vb[v_offset(vc, D, vp, d)]));
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    float const inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t const d = lane + 64u * k;
        if (d < D) item.output[(static_cast<uint64_t>(i) * QH + q) * D + d] = __half_as_ushort(__float2half_rn(o[k] * inv));
    }
}

__global__ __launch_bounds__(kBlock) void prefill_kernel(PoolView P, const kimkv_prefill_item* items,
                                                         const uint32_t* block_prefix, uint32_t item_count,
                                                         uint32_t QH)
{
    __shared__ GroupEntry groups[kMaxGroups];
    __shared__ GenericScratch scratch[4];
    __shared__ uint32_t s_item;
    __shared__ uint32_t s_generic;

    uint32_t const tid = threadIdx.x;
    uint32_t const block = blockIdx.x;
    uint32_t const h = blockIdx.y;
    if (tid == 0) {
        s_item = 0xFFFFFFFFu;
        s_generic = 0;
    }
    __syncthreads();
    for (uint32_t k = tid; k < item_count; k += kBlock) {
        if (block_prefix[k] <= block && block < block_prefix[k + 1]) s_item = k;
    }
    __syncthreads();
    uint32_t const it = s_item;
    if (it == 0xFFFFFFFFu) return;
    kimkv_prefill_item const item = items[it];
    uint32_t const H = P.heads;
    uint32_t const D = P.dim;
    if (h >= H || item.new_tokens == 0 || item.new_tokens > item.token_count || item.descriptors == nullptr
        || item.descriptor_count == 0 || item.query == nullptr || item.output == nullptr || item.layer >= P.layers
        || QH == 0 || QH % H != 0 || D > 256) {
        return;
    }
    PrefillShape const shape = prefill_shape(QH, H, D);
    uint32_t const wave = tid >> 6;
    uint32_t const per_block = 4 * shape.tpw;
    uint32_t const i_block = (block - block_prefix[it]) * per_block;
    uint32_t const i0 = i_block + wave * shape.tpw;          // this wave's first new token
    uint32_t const T0 = item.token_count - item.new_tokens;
    // Keys the whole block needs: [0, T0 + last token of the block].
    uint32_t const last = min(i_block + per_block, item.new_tokens) - 1;
    uint32_t const kend = T0 + last + 1;

    PrefillWave w;
    if (shape.mfma) prefill_wave_init(w, item, h, shape.G, QH, i0);
    bool const wave_has_rows = i0 < item.new_tokens;
    uint32_t const wave_kend = wave_has_rows ? T0 + min(i0 + shape.tpw, item.new_tokens) : 0;   // exclusive

    for (uint32_t s0 = 0; s0 < kend; s0 += kMaxChunk) {
        uint32_t const s1 = min(s0 + kMaxChunk, kend);
        uint32_t const ngroups = (s1 - s0 + 7) / 8;
        for (uint32_t g = tid; g < ngroups; g += kBlock) groups[g] = GroupEntry{nullptr, 0, 0};
        __syncthreads();
        if (shape.mfma) {
            uint32_t const idx0 = find_descriptor_wave(item.descriptors, item.descriptor_count, s0);
            for (uint32_t j = tid; j <= ngroups && idx0 + j < item.descriptor_count; j += kBlock) {
                add_groups(P, item.descriptors[idx0 + j], item.layer, s0, s1, item.token_count, groups, &s_generic);
            }
        }
        __syncthreads();
        if (shape.mfma && s_generic == 0) {
            uint32_t const stop = min(s1, wave_kend);
            for (uint32_t t0 = s0; t0 < stop; t0 += 64) prefill_wave_step(w, groups, s0, s1, t0);
        }
        __syncthreads();
    }
    if (shape.mfma && s_generic == 0) {
        prefill_wave_store(w, item, h, shape.G, QH, i0);
        return;
    }
    // Generic path: this wave's new tokens x the G query heads, one row at a time.
    for (uint32_t i = i0; i < min(i0 + shape.tpw, item.new_tokens); ++i) {
        for (uint32_t g = 0; g < shape.G; ++g) {
            prefill_row_generic(P, item, h, h * shape.G + g, i, QH, &scratch[wave]);
        }
    }
}

}  // namespace
}  // namespace kimkv

using namespace kimkv;

extern "C" {

uint32_t kimkv_prefill_tokens_per_block(const kimkv_storage* storage, uint32_t query_heads)
{
    if (storage == nullptr || query_heads == 0 || storage->layout.kv_heads == 0
        || query_heads % storage->layout.kv_heads != 0) {
        return 0;
    }
    uint32_t const G = query_heads / storage->layout.kv_heads;
    bool const mfma = storage->layout.head_dim == 64 && G <= 16 && 16 % G == 0;
    return 4 * (mfma ? 16 / G : 1);
}

kimkv_status kimkv_paged_prefill_batch(const kimkv_storage* storage, const kimkv_prefill_item* device_items,
                                       const uint32_t* device_block_prefix, uint32_t item_count,
                                       uint32_t total_blocks, uint32_t query_heads, kimkv_stream_t stream)
{
    if (storage == nullptr || device_items == nullptr || device_block_prefix == nullptr || query_heads == 0
        || storage->layout.kv_heads == 0 || query_heads % storage->layout.kv_heads != 0
        || storage->layout.head_dim > 256) {
        return KIMKV_INVALID_ARGUMENT;
    }
    if (total_blocks == 0 || item_count == 0) return KIMKV_OK;
    dim3 const grid(total_blocks, storage->layout.kv_heads);
    prefill_kernel<<<grid, kBlock, 0, native(stream)>>>(pool_view(*storage), device_items, device_block_prefix,
                                                        item_count, query_heads);
    return launch_status();
}

}  // extern "C"
