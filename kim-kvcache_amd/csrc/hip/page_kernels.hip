// page_kernels.hip -- append (with fused partial-tail COW), gather, promotion
// and synthetic fill kernels for gfx950.
//
// Reference kernels these replace (semantics only):
//   copyPageTokensKernel / appendTokensKernel  src/cuda/kv/page_kernels.cu:46-127
//   copyLayerTokensKernel / writeLayerTokenKernel
//                                      src/cuda/attention/paged_decode_kernels.cu:29-99
//   promotionKernel                    src/cuda/kv/page_kernels.cu:129-182
//   gatherKernel                       src/cuda/kv/page_kernels.cu:184-242
#include <hip/hip_runtime.h>

#include "device_common.h"
#include "runtime_internal.h"

namespace kimkv {
namespace {

constexpr unsigned kBlock = 256;
constexpr unsigned kTile = 64;   // tokens per gather/fill tile

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct TokEntry {
    uint16_t* page;
    uint32_t cap;
    uint32_t pt;
};

// Resolves tokens [t0, t0+n) (n <= 64) of a table into LDS entries.  Tokens
// not covered by a valid descriptor get page == nullptr.  All threads of the
// block must call it.
__device__ void build_tile_table(const PoolView& P, const kimkv_block_desc* desc, uint32_t count,
                                 uint32_t t0, uint32_t n, TokEntry* tab, uint32_t* s_idx)
{
    uint32_t const tid = threadIdx.x;
    if (tid < kTile) {
        tab[tid].page = nullptr;
        uint32_t const idx = find_descriptor_wave(desc, count, t0);
        if (tid == 0) {
            *s_idx = idx;
        }
    }
    __syncthreads();
    uint32_t const idx = *s_idx;
    // At most n descriptors overlap the tile, starting at idx.
    if (tid < n && idx + tid < count) {
        kimkv_block_desc const e = desc[idx + tid];
        uint32_t const b = e.logical_token_begin;
        uint32_t const end = b + e.valid_tokens;
        uint32_t const lo = max(b, t0);
        uint32_t const hi = min(end, t0 + n);
        if (lo < hi && e.valid_tokens <= e.page_token_capacity) {
            uint16_t* page = page_base(P, e.kind, e.slot, e.page_token_capacity);
            if (page != nullptr) {
                for (uint32_t t = lo; t < hi; ++t) {
                    tab[t - t0] = TokEntry{page, e.page_token_capacity, t - b};
                }
            }
        }
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Batched append: one block per (job, layer).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void append_kernel(PoolView P, const kimkv_append_job* jobs,
                                                        uint32_t job_count)
{
    if (blockIdx.x >= job_count) return;
    kimkv_append_job const job = jobs[blockIdx.x];
    uint32_t const li = blockIdx.y;
    if (li >= job.layer_count) return;   // a shorter job of a launch sized for the longest
    uint32_t const layer = job.layer_begin + li;
    uint32_t const H = P.heads;
    uint32_t const D = P.dim;
    uint32_t const dcap = pool_tokens(P, job.dst_kind);
    uint16_t* dst = page_base(P, job.dst_kind, job.dst_slot, dcap);
    if (layer >= P.layers || dst == nullptr || static_cast<uint32_t>(job.dst_token) + job.token_count > dcap
        || job.src_key == nullptr || job.src_value == nullptr) {
        report_fault(P, KIMKV_FAULT_APPEND_JOB);
        return;
    }
    uint32_t const tid = threadIdx.x;

    if (job.cow_tokens != 0) {
        uint32_t const scap = pool_tokens(P, job.cow_kind);
        uint16_t const* src = page_base(P, job.cow_kind, job.cow_slot, scap);
        uint32_t const n = job.cow_tokens;
        if (src != nullptr && n <= scap && n <= dcap && n <= job.dst_token) {
            uint32_t const per_head = n * D;
            for (uint32_t i = tid; i < H * per_head; i += kBlock) {
                uint32_t const h = i / per_head;
                uint32_t const rem = i - h * per_head;
                uint32_t const t = rem / D;
                uint32_t const d = rem - t * D;
                uint64_t const sh = head_block(P, scap, layer, h);
                uint64_t const dh = head_block(P, dcap, layer, h);
                dst[dh + k_offset(dcap, D, t, d)] = src[sh + k_offset(scap, D, t, d)];
                dst[dh + v_offset(dcap, D, t, d)] = src[sh + v_offset(scap, D, t, d)];
            }
        }
        __syncthreads();
    }

    uint32_t const HD = H * D;
    uint32_t const total = job.token_count * HD;
    uint64_t const layer_off = static_cast<uint64_t>(li) * job.src_layer_stride;
    const uint16_t* sk = job.src_key + layer_off;
    const uint16_t* sv = job.src_value + layer_off;
    uint32_t const stride = job.src_token_stride;
    bool const src_aligned = (D & 7u) == 0 && (stride & 7u) == 0
        && ((reinterpret_cast<uintptr_t>(sk) | reinterpret_cast<uintptr_t>(sv)) & 15u) == 0;
    if (src_aligned) {
        // K: 16-byte pieces of 8 dims of one token (contiguous in source and page).
        uint32_t const dchunks = D / 8;
        uint32_t const kchunks = job.token_count * H * dchunks;
        for (uint32_t i = tid; i < kchunks; i += kBlock) {
            uint32_t const t = i / (H * dchunks);
            uint32_t const rem = i - t * (H * dchunks);
            uint32_t const h = rem / dchunks;
            uint32_t const dc = rem - h * dchunks;
            u32x4_t const v = *reinterpret_cast<const u32x4_t*>(sk + static_cast<uint64_t>(t) * stride + h * D + dc * 8);
            *reinterpret_cast<u32x4_t*>(dst + head_block(P, dcap, layer, h)
                                        + k_offset(dcap, D, job.dst_token + t, dc * 8)) = v;
        }
        // V^T: 16-byte pieces of 8 tokens of one dim when the tokens sit in
        // 8-aligned groups of the page, else one element at a time.
        bool const v_groups = (job.token_count & 7u) == 0 && (job.dst_token & 7u) == 0 && (dcap & 7u) == 0;
        if (v_groups) {
            uint32_t const vchunks = (job.token_count / 8) * HD;
            for (uint32_t i = tid; i < vchunks; i += kBlock) {
                uint32_t const g = i / HD;
                uint32_t const r = i - g * HD;
                uint32_t const h = r / D;
                uint32_t const d = r - h * D;
                const uint16_t* src = sv + static_cast<uint64_t>(8 * g) * stride + r;
                u32x4_t w;
#pragma unroll
                for (uint32_t j = 0; j < 4; ++j) {
                    w[j] = static_cast<uint32_t>(src[static_cast<uint64_t>(2 * j) * stride])
                        | (static_cast<uint32_t>(src[static_cast<uint64_t>(2 * j + 1) * stride]) << 16);
                }
                *reinterpret_cast<u32x4_t*>(dst + head_block(P, dcap, layer, h)
                                            + v_offset(dcap, D, job.dst_token + 8 * g, d)) = w;
            }
            return;
        }
        for (uint32_t i = tid; i < total; i += kBlock) {
            uint32_t const t = i / HD;
            uint32_t const rem = i - t * HD;
            uint32_t const h = rem / D;
            uint32_t const d = rem - h * D;
            dst[head_block(P, dcap, layer, h) + v_offset(dcap, D, job.dst_token + t, d)] =
                sv[static_cast<uint64_t>(t) * stride + rem];
        }
        return;
    }
    for (uint32_t i = tid; i < total; i += kBlock) {
        uint32_t const t = i / HD;
        uint32_t const rem = i - t * HD;
        uint32_t const h = rem / D;
        uint32_t const d = rem - h * D;
        uint64_t const so = layer_off + static_cast<uint64_t>(t) * job.src_token_stride + rem;
        uint64_t const dh = head_block(P, dcap, layer, h);
        uint32_t const pt = job.dst_token + t;
        dst[dh + k_offset(dcap, D, pt, d)] = job.src_key[so];
        dst[dh + v_offset(dcap, D, pt, d)] = job.src_value[so];
    }
}

// ---------------------------------------------------------------------------
// Gather: block = (64-token tile, group of layers); output [L][2][T][H][D].
// Fast path (full tile whose 8-token groups each sit 8-aligned in one page,
// D % 8 == 0): every thread issues all its 16-byte non-temporal loads before
// any store.  K rows are copied straight; V^T is transposed through LDS
// (16-byte chunks of 8 tokens of one dim row in, 16-byte chunks of 8 dims of
// one token out; the chunk column is XOR-swizzled by the token's group so the
// scattered 2-byte writes of one instruction spread over the banks).  Other
// tiles take the element-wise path.
// ---------------------------------------------------------------------------
constexpr unsigned kRowChunk = 256;            // V rows (head x dim) per pass
constexpr unsigned kStageRow = kRowChunk + 8;  // u16 per staged token row (16-byte multiple)
constexpr unsigned kGatherLoads = 8;           // 16-byte loads in flight per thread

typedef const __attribute__((address_space(1))) u32x4_t global_u32x4_t;
typedef __attribute__((address_space(1))) u32x4_t global_u32x4_out_t;

__device__ inline u32x4_t load16_nt(const uint16_t* p)
{
    return __builtin_nontemporal_load((global_u32x4_t*)(p));
}

__device__ inline void store16_nt(uint16_t* p, u32x4_t v)
{
    __builtin_nontemporal_store(v, (global_u32x4_out_t*)(p));
}

__device__ inline uint32_t stage_col(uint32_t t, uint32_t r)
{
    return (((r >> 3) ^ ((t >> 3) & 3u)) << 3) | (r & 7u);
}

// K rows of one (tile, layer): straight 16-byte copies, all loads first.
__device__ inline void gather_k_fast(const PoolView& P, const TokEntry* tab, uint32_t layer, uint16_t* out_base)
{
    uint32_t const tid = threadIdx.x;
    uint32_t const D = P.dim;
    uint32_t const dchunks = D / 8;
    uint32_t const per_token = P.heads * dchunks;
    uint32_t const total = kTile * per_token;
    for (uint32_t base = 0; base < total; base += kBlock * kGatherLoads) {
        u32x4_t v[kGatherLoads];
#pragma unroll
        for (uint32_t k = 0; k < kGatherLoads; ++k) {
            uint32_t const i = base + k * kBlock + tid;
            if (i < total) {
                uint32_t const t = i / per_token;
                uint32_t const c = i - t * per_token;
                uint32_t const h = c / dchunks;
                TokEntry const e = tab[t];
                v[k] = load16_nt(e.page + head_block(P, e.cap, layer, h) + k_offset(e.cap, D, e.pt, (c - h * dchunks) * 8));
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < kGatherLoads; ++k) {
            uint32_t const i = base + k * kBlock + tid;
            if (i < total) store16_nt(out_base + static_cast<uint64_t>(i) * 8, v[k]);
        }
    }
}

// V^T rows of one (tile, layer) transposed through LDS.
__device__ inline void gather_v_fast(const PoolView& P, const TokEntry* tab, uint32_t layer, uint16_t* out_base,
                                     uint16_t* stage)
{
    uint32_t const tid = threadIdx.x;
    uint32_t const D = P.dim;
    uint32_t const HD = P.heads * D;
    for (uint32_t r0 = 0; r0 < HD; r0 += kRowChunk) {
        uint32_t const rows = min(kRowChunk, HD - r0);
        uint32_t const chunks = rows * 8;   // (row, 8-token group) pairs
        // Chunk q: group (q & 3) + 4 * ((q >> 2) / rows), row (q >> 2) % rows: four consecutive
        // lanes read one 64-byte dim row of a 32-token V^T panel.
        for (uint32_t base = 0; base < chunks; base += kBlock * kGatherLoads) {
            u32x4_t v[kGatherLoads];
#pragma unroll
            for (uint32_t k = 0; k < kGatherLoads; ++k) {
                uint32_t const q = base + k * kBlock + tid;
                if (q < chunks) {
                    uint32_t const rr = (q >> 2) % rows;
                    uint32_t const g = (q & 3u) + 4u * ((q >> 2) / rows);
                    uint32_t const r = r0 + rr;
                    uint32_t const h = r / D;
                    TokEntry const e = tab[8 * g];
                    v[k] = load16_nt(e.page + head_block(P, e.cap, layer, h) + v_offset(e.cap, D, e.pt, r - h * D));
                }
            }
#pragma unroll
            for (uint32_t k = 0; k < kGatherLoads; ++k) {
                uint32_t const q = base + k * kBlock + tid;
                if (q < chunks) {
                    uint32_t const rr = (q >> 2) % rows;
                    uint32_t const g = (q & 3u) + 4u * ((q >> 2) / rows);
#pragma unroll
                    for (uint32_t j = 0; j < 8; ++j) {
                        uint32_t const t = 8 * g + j;
                        uint32_t const word = v[k][j >> 1];
                        stage[t * kStageRow + stage_col(t, rr)] =
                            static_cast<uint16_t>((j & 1u) ? (word >> 16) : (word & 0xFFFFu));
                    }
                }
            }
        }
        __syncthreads();
        uint32_t const per_token = rows / 8;
        for (uint32_t i = tid; i < kTile * per_token; i += kBlock) {
            uint32_t const t = i / per_token;
            uint32_t const c = i - t * per_token;
            u32x4_t const w = *reinterpret_cast<const u32x4_t*>(&stage[t * kStageRow + stage_col(t, c * 8)]);
            store16_nt(out_base + static_cast<uint64_t>(t) * HD + r0 + c * 8, w);
        }
        __syncthreads();
    }
}

// One (tile, layer) with H * D == kRowChunk: the K and V^T loads of the
// layer (8 + 8 per thread) are all in flight before the first store.
__device__ inline void gather_kv_fast(const PoolView& P, const TokEntry* tab, uint32_t layer, uint16_t* k_base,
                                      uint16_t* v_base, uint16_t* stage)
{
    constexpr uint32_t rows = kRowChunk;
    constexpr uint32_t per = kTile * rows / 8 / kBlock;   // 16-byte chunks per thread, each of K and V
    uint32_t const tid = threadIdx.x;
    uint32_t const D = P.dim;
    uint32_t const dchunks = D / 8;
    constexpr uint32_t per_token = rows / 8;
    u32x4_t kv[per], vv[per];
#pragma unroll
    for (uint32_t k = 0; k < per; ++k) {
        uint32_t const i = k * kBlock + tid;
        uint32_t const t = i / per_token;
        uint32_t const c = i - t * per_token;
        uint32_t const h = c / dchunks;
        TokEntry const e = tab[t];
        kv[k] = load16_nt(e.page + head_block(P, e.cap, layer, h) + k_offset(e.cap, D, e.pt, (c - h * dchunks) * 8));
    }
#pragma unroll
    for (uint32_t k = 0; k < per; ++k) {
        uint32_t const q = k * kBlock + tid;
        uint32_t const rr = (q >> 2) % rows;
        uint32_t const g = (q & 3u) + 4u * ((q >> 2) / rows);
        uint32_t const h = rr / D;
        TokEntry const e = tab[8 * g];
        vv[k] = load16_nt(e.page + head_block(P, e.cap, layer, h) + v_offset(e.cap, D, e.pt, rr - h * D));
    }
#pragma unroll
    for (uint32_t k = 0; k < per; ++k) store16_nt(k_base + static_cast<uint64_t>(k * kBlock + tid) * 8, kv[k]);
#pragma unroll
    for (uint32_t k = 0; k < per; ++k) {
        uint32_t const q = k * kBlock + tid;
        uint32_t const rr = (q >> 2) % rows;
        uint32_t const g = (q & 3u) + 4u * ((q >> 2) / rows);
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            uint32_t const t = 8 * g + j;
            uint32_t const word = vv[k][j >> 1];
            stage[t * kStageRow + stage_col(t, rr)] = static_cast<uint16_t>((j & 1u) ? (word >> 16) : (word & 0xFFFFu));
        }
    }
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < per; ++k) {
        uint32_t const i = k * kBlock + tid;
        uint32_t const t = i / per_token;
        uint32_t const c = i - t * per_token;
        u32x4_t const w = *reinterpret_cast<const u32x4_t*>(&stage[t * kStageRow + stage_col(t, c * 8)]);
        store16_nt(v_base + static_cast<uint64_t>(t) * rows + c * 8, w);
    }
    __syncthreads();
}

// Block = (64-token tile, group of layers_per_block layers): the tile's page
// table is resolved once for all its layers and both components.
__global__ __launch_bounds__(kBlock) void gather_kernel(PoolView P, const kimkv_block_desc* desc,
                                                        uint32_t count, uint32_t T, uint32_t layers_per_block,
                                                        uint16_t* out)
{
    __shared__ TokEntry tab[kTile];
    __shared__ uint32_t s_idx;
    __shared__ __align__(16) uint16_t stage[kTile * kStageRow];

    uint32_t const t0 = blockIdx.x * kTile;
    uint32_t const n = min(kTile, T - t0);
    build_tile_table(P, desc, count, t0, n, tab, &s_idx);

    uint32_t const D = P.dim;
    uint32_t const HD = P.heads * D;
    uint32_t const tid = threadIdx.x;
    uint32_t const l0 = blockIdx.y * layers_per_block;
    uint32_t const l1 = min(P.layers, l0 + layers_per_block);

    int group_ok = 1;
    if (tid < kTile / 8) {
        TokEntry const a = tab[8 * tid];
        TokEntry const b = tab[8 * tid + 7];
        group_ok = a.page != nullptr && b.page == a.page && (a.pt & 7u) == 0 && b.pt == a.pt + 7
            && (a.cap & 7u) == 0;
    }
    bool const fast = __syncthreads_and(group_ok) && n == kTile && (D & 7u) == 0;

    for (uint32_t layer = l0; layer < l1; ++layer) {
        uint16_t* k_base = out + (static_cast<uint64_t>(layer * 2) * T + t0) * HD;
        uint16_t* v_base = out + (static_cast<uint64_t>(layer * 2 + 1) * T + t0) * HD;
        if (fast && HD == kRowChunk) {
            gather_kv_fast(P, tab, layer, k_base, v_base, stage);
            continue;
        }
        if (fast) {
            gather_k_fast(P, tab, layer, k_base);
            gather_v_fast(P, tab, layer, v_base, stage);
            continue;
        }
        // Element-wise path: partial tiles, unaligned groups, D % 8 != 0.
        for (uint32_t i = tid; i < n * HD; i += kBlock) {
            uint32_t const t = i / HD;
            uint32_t const r = i - t * HD;
            TokEntry const e = tab[t];
            if (e.page == nullptr) continue;
            uint32_t const h = r / D;
            uint32_t const d = r - h * D;
            uint16_t const* hb = e.page + head_block(P, e.cap, layer, h);
            k_base[i] = hb[k_offset(e.cap, D, e.pt, d)];
            v_base[i] = hb[v_offset(e.cap, D, e.pt, d)];
        }
    }
}

// ---------------------------------------------------------------------------
// Batched promotion: block = (job, layer).  Extent token t <- micro page t/8.
// ---------------------------------------------------------------------------
// One workgroup per patch: the range is copied as 32-bit words (a
// descriptor is 5 words), so a one-entry patch is a single wave's loads.
__global__ __launch_bounds__(kBlock) void patch_descriptors_kernel(const kimkv_descriptor_patch* patches,
                                                                   const kimkv_block_desc* descriptors)
{
    static_assert(sizeof(kimkv_block_desc) == 5 * sizeof(uint32_t), "descriptor is five words");
    kimkv_descriptor_patch const p = patches[blockIdx.x];
    uint32_t const words = p.count * 5u;
    auto const* src = reinterpret_cast<const uint32_t*>(descriptors + p.source);
    auto* dst = reinterpret_cast<uint32_t*>(p.table + p.first);
    for (uint32_t w = threadIdx.x; w < words; w += kBlock) dst[w] = src[w];
}

__global__ __launch_bounds__(kBlock) void promote_kernel(PoolView P, const kimkv_promotion_job* jobs,
                                                         uint32_t job_count)
{
    if (blockIdx.x >= job_count) return;
    kimkv_promotion_job const job = jobs[blockIdx.x];
    uint32_t const layer = blockIdx.y;
    uint32_t const mt = P.micro_tokens;
    uint32_t const et = P.extent_tokens;
    uint16_t* dst = page_base(P, KIMKV_PAGE_EXTENT, job.extent_slot, et);
    uint16_t const* src[8];
    bool ok = mt * 8 == et && layer < P.layers && dst != nullptr;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        src[k] = page_base(P, KIMKV_PAGE_MICRO, job.micro_slots[k], mt);
        ok = ok && src[k] != nullptr;
    }
    if (!ok) {
        report_fault(P, KIMKV_FAULT_PROMOTION_JOB);
        return;
    }
    uint32_t const H = P.heads;
    uint32_t const D = P.dim;
    uint32_t const tid = threadIdx.x;
    if ((D & 7u) == 0 && mt == 8) {
        uint32_t const dchunks = D / 8;
        // K: (h, t, dc) 16-byte chunks.
        uint32_t const kchunks = H * et * dchunks;
        for (uint32_t i = tid; i < kchunks; i += kBlock) {
            uint32_t const h = i / (et * dchunks);
            uint32_t const rem = i - h * et * dchunks;
            uint32_t const t = rem / dchunks;
            uint32_t const dc = rem - t * dchunks;
            uint4 const v = *reinterpret_cast<uint4 const*>(
                src[t >> 3] + head_block(P, mt, layer, h) + k_offset(mt, D, t & 7u, dc * 8));
            *reinterpret_cast<uint4*>(dst + head_block(P, et, layer, h) + k_offset(et, D, t, dc * 8)) = v;
        }
        // V^T: (h, d, k) -- micro row d (8 tokens, 16 bytes) -> extent row d at 8k.
        uint32_t const vchunks = H * D * 8;
        for (uint32_t i = tid; i < vchunks; i += kBlock) {
            uint32_t const h = i / (D * 8);
            uint32_t const rem = i - h * D * 8;
            uint32_t const d = rem / 8;
            uint32_t const k = rem & 7u;
            uint4 const v = *reinterpret_cast<uint4 const*>(
                src[k] + head_block(P, mt, layer, h) + v_offset(mt, D, 0, d));
            *reinterpret_cast<uint4*>(dst + head_block(P, et, layer, h) + v_offset(et, D, 8 * k, d)) = v;
        }
        return;
    }
    uint32_t const total = H * et * D;
    for (uint32_t i = tid; i < total; i += kBlock) {
        uint32_t const h = i / (et * D);
        uint32_t const rem = i - h * et * D;
        uint32_t const t = rem / D;
        uint32_t const d = rem - t * D;
        uint16_t const* s = src[t / mt];
        uint32_t const st = t % mt;
        uint64_t const sh = head_block(P, mt, layer, h);
        uint64_t const dh = head_block(P, et, layer, h);
        dst[dh + k_offset(et, D, t, d)] = s[sh + k_offset(mt, D, st, d)];
        dst[dh + v_offset(et, D, t, d)] = s[sh + v_offset(mt, D, st, d)];
    }
}

// ---------------------------------------------------------------------------
// Synthetic fill of a table's pages: block = (64-token tile, layer, component).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void fill_table_kernel(PoolView P, const kimkv_block_desc* desc,
                                                            uint32_t count, uint32_t token_begin,
                                                            uint32_t token_end, uint64_t seed,
                                                            uint32_t stream_id)
{
    __shared__ TokEntry tab[kTile];
    __shared__ uint32_t s_idx;
    uint32_t const t0 = token_begin + blockIdx.x * kTile;
    uint32_t const n = min(kTile, token_end - t0);
    uint32_t const layer = blockIdx.y;
    uint32_t const comp = blockIdx.z;
    build_tile_table(P, desc, count, t0, n, tab, &s_idx);
    uint32_t const D = P.dim;
    uint32_t const HD = P.heads * D;
    uint32_t const tid = threadIdx.x;

    if (comp == 0) {
        for (uint32_t i = tid; i < n * HD; i += kBlock) {
            uint32_t const t = i / HD;
            uint32_t const r = i - t * HD;
            TokEntry const e = tab[t];
            if (e.page == nullptr) continue;
            uint32_t const h = r / D;
            uint32_t const d = r - h * D;
            e.page[head_block(P, e.cap, layer, h) + k_offset(e.cap, D, e.pt, d)] =
                synth_f16(seed, kv_row(stream_id, layer, 0, t0 + t), r);
        }
        return;
    }
    // V^T: thread per (row, token group of 8) with 16-byte stores when aligned.
    uint32_t const groups = (n + 7) / 8;
    for (uint32_t i = tid; i < HD * groups; i += kBlock) {
        uint32_t const r = i / groups;
        uint32_t const g = i - r * groups;
        uint32_t const h = r / D;
        uint32_t const d = r - h * D;
        uint32_t const tb = g * 8;
        uint32_t const te = min(tb + 8, n);
        TokEntry const e = tab[tb];
        bool const vec = te == tb + 8 && e.page != nullptr && (e.pt & 7u) == 0 && (e.cap & 7u) == 0
            && tab[tb + 7].page == e.page && tab[tb + 7].pt == e.pt + 7;
        if (vec) {
            uint32_t w[4];
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                uint32_t const lo = synth_f16(seed, kv_row(stream_id, layer, 1, t0 + tb + 2 * j), r);
                uint32_t const hi = synth_f16(seed, kv_row(stream_id, layer, 1, t0 + tb + 2 * j + 1), r);
                w[j] = lo | (hi << 16);
            }
            *reinterpret_cast<uint4*>(e.page + head_block(P, e.cap, layer, h) + v_offset(e.cap, D, e.pt, d)) =
                make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            for (uint32_t t = tb; t < te; ++t) {
                TokEntry const f = tab[t];
                if (f.page == nullptr) continue;
                f.page[head_block(P, f.cap, layer, h) + v_offset(f.cap, D, f.pt, d)] =
                    synth_f16(seed, kv_row(stream_id, layer, 1, t0 + t), r);
            }
        }
    }
}

__global__ __launch_bounds__(kBlock) void fill_rows_kernel(uint16_t* out, uint64_t count, uint64_t seed,
                                                           uint64_t row0, uint32_t cols)
{
    uint64_t const stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < count; i += stride) {
        out[i] = synth_f16(seed, row0 + i / cols, static_cast<uint32_t>(i % cols));
    }
}

// Contiguous K/V block [layers][2][tokens][cols]: the row of (l, c, t) is
// kv_row(stream_id, l, c, token0 + t).
__global__ __launch_bounds__(kBlock) void fill_kv_kernel(uint16_t* out, uint32_t layers, uint32_t tokens,
                                                         uint32_t cols, uint64_t seed, uint32_t stream_id,
                                                         uint32_t token0)
{
    uint64_t const per_block = static_cast<uint64_t>(tokens) * cols;
    uint64_t const count = per_block * 2u * layers;
    uint64_t const stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < count; i += stride) {
        uint64_t const lc = i / per_block;
        uint64_t const r = i - lc * per_block;
        uint32_t const t = static_cast<uint32_t>(r / cols);
        uint32_t const col = static_cast<uint32_t>(r - static_cast<uint64_t>(t) * cols);
        out[i] = synth_f16(seed, kv_row(stream_id, static_cast<uint32_t>(lc >> 1), static_cast<uint32_t>(lc & 1u),
                                        token0 + t),
                           col);
    }
}

}  // namespace
}  // namespace kimkv

using namespace kimkv;

extern "C" {

kimkv_status kimkv_append_batch(const kimkv_storage* storage, const kimkv_append_job* device_jobs,
                                uint32_t job_count, uint32_t max_layer_count, kimkv_stream_t stream)
{
    if (storage == nullptr || (job_count != 0 && device_jobs == nullptr)) return KIMKV_INVALID_ARGUMENT;
    if (job_count == 0 || max_layer_count == 0) return KIMKV_OK;
    if (max_layer_count > storage->layout.layers || job_count > 0x7FFFFFFFu) return KIMKV_INVALID_ARGUMENT;
    dim3 const grid(job_count, max_layer_count);
    void* start = nullptr;
    kernel_timing_begin(TimedKernel::Append, native(stream), &start);
    append_kernel<<<grid, kBlock, 0, native(stream)>>>(pool_view(*storage), device_jobs, job_count);
    kimkv_status const status = launch_status();
    kernel_timing_end(TimedKernel::Append, native(stream), start);
    return status;
}

kimkv_status kimkv_gather(const kimkv_storage* storage, const kimkv_block_desc* device_descriptors,
                          uint32_t descriptor_count, uint32_t total_tokens, uint16_t* device_output,
                          kimkv_stream_t stream)
{
    if (storage == nullptr || device_descriptors == nullptr || device_output == nullptr
        || descriptor_count == 0 || total_tokens == 0) {
        return KIMKV_INVALID_ARGUMENT;
    }
    // Enough workgroups to fill the chip (~8 per CU) with as few table
    // resolutions as possible: layers are grouped per workgroup.
    uint32_t const tiles = ceil_div(total_tokens, kTile);
    uint32_t const L = storage->layout.layers;
    uint32_t per = 1;
    while (per < L && static_cast<uint64_t>(tiles) * ceil_div(L, per * 2) >= 2048) per *= 2;
    dim3 const grid(tiles, ceil_div(L, per));
    gather_kernel<<<grid, kBlock, 0, native(stream)>>>(pool_view(*storage), device_descriptors,
                                                       descriptor_count, total_tokens, per, device_output);
    return launch_status();
}

kimkv_status kimkv_promote_batch(const kimkv_storage* storage, const kimkv_promotion_job* device_jobs,
                                 uint32_t job_count, kimkv_stream_t stream)
{
    if (storage == nullptr || (job_count != 0 && device_jobs == nullptr)) return KIMKV_INVALID_ARGUMENT;
    if (job_count == 0) return KIMKV_OK;
    if (static_cast<uint32_t>(storage->micro_tokens) * 8 != storage->extent_tokens) return KIMKV_INVALID_ARGUMENT;
    dim3 const grid(job_count, storage->layout.layers);
    promote_kernel<<<grid, kBlock, 0, native(stream)>>>(pool_view(*storage), device_jobs, job_count);
    return launch_status();
}

kimkv_status kimkv_patch_descriptors(const kimkv_descriptor_patch* patches, uint32_t patch_count,
                                     const kimkv_block_desc* descriptors, kimkv_stream_t stream)
{
    if (patch_count == 0) return KIMKV_OK;
    if (patches == nullptr || descriptors == nullptr) return KIMKV_INVALID_ARGUMENT;
    patch_descriptors_kernel<<<patch_count, kBlock, 0, native(stream)>>>(patches, descriptors);
    return launch_status();
}

kimkv_status kimkv_fill_table(const kimkv_storage* storage, const kimkv_block_desc* device_descriptors,
                              uint32_t descriptor_count, uint32_t token_begin, uint32_t token_end,
                              uint64_t seed, uint32_t stream_id, kimkv_stream_t stream)
{
    if (storage == nullptr || device_descriptors == nullptr || descriptor_count == 0 || token_end < token_begin) {
        return KIMKV_INVALID_ARGUMENT;
    }
    if (token_end == token_begin) return KIMKV_OK;
    dim3 const grid(ceil_div(token_end - token_begin, kTile), storage->layout.layers, 2);
    fill_table_kernel<<<grid, kBlock, 0, native(stream)>>>(pool_view(*storage), device_descriptors,
                                                           descriptor_count, token_begin, token_end, seed,
                                                           stream_id);
    return launch_status();
}

kimkv_status kimkv_fill_rows(uint16_t* device_out, uint64_t count, uint64_t seed, uint64_t row0,
                             uint32_t cols, kimkv_stream_t stream)
{
    if (device_out == nullptr || cols == 0) return KIMKV_INVALID_ARGUMENT;
    if (count == 0) return KIMKV_OK;
    uint64_t const blocks64 = (count + kBlock - 1) / kBlock;
    unsigned const blocks = static_cast<unsigned>(blocks64 < 65536 ? blocks64 : 65536);
    fill_rows_kernel<<<blocks, kBlock, 0, native(stream)>>>(device_out, count, seed, row0, cols);
    return launch_status();
}

kimkv_status kimkv_fill_kv(uint16_t* device_out, uint32_t layers, uint32_t tokens, uint32_t cols, uint64_t seed,
                           uint32_t stream_id, uint32_t token0, kimkv_stream_t stream)
{
    if (device_out == nullptr || cols == 0 || static_cast<uint64_t>(token0) + tokens > (1ull << 32)) {
        return KIMKV_INVALID_ARGUMENT;
    }
    uint64_t const count = static_cast<uint64_t>(layers) * 2u * tokens * cols;
    if (count == 0) return KIMKV_OK;
    uint64_t const blocks64 = (count + kBlock - 1) / kBlock;
    unsigned const blocks = static_cast<unsigned>(blocks64 < 65536 ? blocks64 : 65536);
    fill_kv_kernel<<<blocks, kBlock, 0, native(stream)>>>(device_out, layers, tokens, cols, seed, stream_id, token0);
    return launch_status();
}

}  // extern "C"
