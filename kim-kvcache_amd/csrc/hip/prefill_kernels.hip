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
// Work: block = (item, KV head, 8 * tpw new tokens), 4 waves, each wave two
// 16-column MFMA blocks whose columns are tpw tokens x G query heads
// (tpw = 16 / G; TinyLlama's G = 8 gives 16 tokens = 256 query rows per
// block).  The block walks the keys up to its last token's position in
// 64-key tiles: all 256 threads load a tile's K and V^T (16 KiB) once into a
// double-buffered, bank-swizzled LDS stage, and every wave runs
// S^T = K.Q^T and O^T += V^T.P^T for its 32 columns on
// v_mfma_f32_16x16x32_f16 (same operand layout as the decode kernel), with an
// online softmax in base 2, fp32 accumulation and fp16 output, while the next
// tile's loads are in flight.  Keys past a column's causal limit are masked
// per column (only on the diagonal tiles).  The group table (8-token groups
// of the key range, resolved to K and V^T pointers of the block's head) is
// built in LDS one 4096-key segment at a time.
// Tables that do not keep 8-token groups aligned, head dims other than 64 and
// group sizes that do not divide 16 take a one-row-at-a-time generic path.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <vector>

#include "attention_common.h"
#include "device_common.h"
#include "runtime_internal.h"

namespace kimkv {
namespace {

constexpr unsigned kBlock = 256;   // 4 waves
constexpr unsigned kWaves = kBlock / 64;
constexpr unsigned kColBlocks = 2;  // 16-column MFMA blocks per wave
constexpr unsigned kTileKeys = 64;
constexpr float kLazyRescaleLog2 = 8.0f;

struct PrefillShape {
    uint32_t tpw;        // new tokens per 16-column block
    uint32_t G;          // query heads per KV head
    bool mfma;           // D == 64 and G divides 16
};

__host__ __device__ inline PrefillShape prefill_shape(uint32_t QH, uint32_t H, uint32_t D)
{
    uint32_t const G = QH / H;
    bool const mfma = D == 64 && G >= 1 && G <= 16 && 16 % G == 0;
    return PrefillShape{mfma ? 16 / G : 1, G, mfma};
}

__host__ __device__ inline uint32_t prefill_block_tokens(PrefillShape s)
{
    return s.mfma ? kWaves * kColBlocks * s.tpw : kWaves;
}

// One 64-key tile of one KV head (D = 64) staged in LDS, in 16-byte units:
//   K   unit (key t, dim octet o) at t * 8 + (o ^ k_swizzle(t))
//   V^T unit (dim d, key octet c) at d * 8 + (c ^ (d & 7))
// The swizzles put the eight 16-byte reads that one LDS cycle serves (lanes
// 8j .. 8j + 7 of an MFMA operand read) on eight different bank groups.
struct KvTile {
    half8_t k[kTileKeys * 8];
    half8_t v[64 * 8];
};

__device__ inline uint32_t k_swizzle(uint32_t t) { return (t & 3u) | (((t >> 3) & 1u) << 2); }
__device__ inline uint32_t k_unit(uint32_t t, uint32_t o) { return t * 8u + (o ^ k_swizzle(t)); }
__device__ inline uint32_t v_unit(uint32_t d, uint32_t c) { return d * 8u + (c ^ (d & 7u)); }

// Keys per group-table segment of the prefill kernel (multiple of 64).
constexpr unsigned kSegmentKeys = 4096;
constexpr unsigned kSegmentGroups = kSegmentKeys / 8;

// One 8-key group of the segment resolved for the block's layer and KV head:
// k points at the group's first key in K panel 0 (panel 1, dims 32..63, is
// kpanel elements further), v at the group's first key in V^T row 0 (dim d is
// d * vw elements further).
struct HeadGroup {
    const uint16_t* k;
    const uint16_t* v;
    uint32_t kpanel;
    uint32_t vw;
    uint64_t pad;
};

// Records the 8-key groups of [c0, c1) that entry `e` covers, for layer /
// head.  An entry whose pages do not keep 8-token groups aligned (or that
// names no page of the storage) switches the block to the generic path.
__device__ inline void add_head_groups(const PoolView& P, kimkv_block_desc const& e, uint32_t layer, uint32_t h,
                                       uint32_t c0, uint32_t c1, uint32_t T, HeadGroup* groups, uint32_t* s_generic)
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
    const uint16_t* hb = page + head_block(P, cap, layer, h);
    uint32_t const vw = v_width(cap);
    for (uint32_t g = (lo - c0) >> 3; g < (hi - c0 + 7) >> 3; ++g) {
        uint32_t const pt0 = c0 + 8 * g - b;
        groups[g] = HeadGroup{hb + k_offset(cap, 64, pt0, 0), hb + v_offset(cap, 64, pt0, 0), cap * 32u, vw, 0};
    }
}

// A thread's share of one tile in flight: two K units and two V^T units.
//   K unit j:   chunk c = tid + 256 j -> group c / 64, panel (c / 32) % 2, key (c / 4) % 8, octet c % 4
//               (a wave reads one 8-key group: two contiguous 512-byte runs of the page)
//   V^T unit j: key octet 4 j + tid % 4, dim tid / 4
//               (four consecutive lanes read one dim row of a 32-key V^T panel: 64 contiguous bytes)
struct TileLoad {
    half8_t k[2];
    half8_t v[2];
};

// A wave-uniform 64-bit value in SGPRs.  readfirstlane returns int: each
// half goes through uint32_t so that the low half is not sign-extended.
__device__ __attribute__((always_inline)) inline uint64_t uniform_u64(uint64_t x)
{
    uint32_t const lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x)));
    uint32_t const hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x >> 32)));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// kFull: all 64 keys of the tile are below nvalid and every group of the
// segment names a page, so no lane needs a check.  A K unit's group (c / 64)
// is the same for the whole wave: its base goes to SGPRs and each lane adds a
// 32-bit offset (panel (tid / 32) % 2, key (tid / 4) % 8, octet tid % 4, the
// same for both units).
template <bool kFull>
__device__ inline void tile_fetch(TileLoad& r, const HeadGroup* groups, uint32_t tg, uint32_t nvalid, uint32_t tid)
{
    half8_t const zero8 = {};
    uint32_t const tk = (tid >> 2) & 7u;
    uint32_t const k_off = tk * 64u + (tid & 3u) * 16u;
    uint32_t const k_panel = (tid >> 5) & 1u;
#pragma unroll
    for (uint32_t j = 0; j < 2; ++j) {
        uint32_t const g = (tid >> 6) + kWaves * j;
        if (kFull || 8 * g + tk < nvalid) {
            HeadGroup const e = groups[tg + g];
            uint64_t const kb = uniform_u64(reinterpret_cast<uintptr_t>(e.k));
            uint32_t const off = k_off + k_panel * static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(e.kpanel)) * 2u;
            r.k[j] = zero8;
            if (kFull || kb != 0) {
                r.k[j] = __builtin_nontemporal_load(reinterpret_cast<const global_half8_t*>(kb + off));
            }
        } else {
            r.k[j] = zero8;
        }
        uint32_t const ko = 4 * j + (tid & 3u);
        if (kFull) {
            HeadGroup const e = groups[tg + ko];
            r.v[j] = load_half8_stream(e.v + (tid >> 2) * e.vw);
        } else {
            r.v[j] = zero8;
            if (8 * ko < nvalid) {
                HeadGroup const e = groups[tg + ko];
                if (e.v != nullptr) {
                    r.v[j] = load_half8_stream(e.v + (tid >> 2) * e.vw);
                    if (8 * ko + 8 > nvalid) {
                        uint32_t const keep = nvalid - 8 * ko;
#pragma unroll
                        for (uint32_t q = 0; q < 8; ++q) {
                            if (q >= keep) r.v[j][q] = static_cast<_Float16>(0.0f);
                        }
                    }
                }
            }
        }
    }
}

__device__ inline void tile_store(KvTile& t, const TileLoad& r, uint32_t tid)
{
#pragma unroll
    for (uint32_t j = 0; j < 2; ++j) {
        uint32_t const c = tid + kBlock * j;
        uint32_t const key = 8 * (c >> 6) + ((c >> 2) & 7u);
        t.k[k_unit(key, 4 * ((c >> 5) & 1u) + (c & 3u))] = r.k[j];
        t.v[v_unit(tid >> 2, 4 * j + (tid & 3u))] = r.v[j];
    }
}

// Cross-row exchanges of a wave64 on the VALU (v_permlane16/32_swap): the
// value of lane l ^ 16 and of lane l ^ 32.
__device__ inline float xor16(float v)
{
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((threadIdx.x & 16u) ? r[0] : r[1]);
}

__device__ inline float xor32(float v)
{
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((threadIdx.x & 32u) ? r[0] : r[1]);
}

// One wave of the fast path: kColBlocks column blocks of 16 columns, each
// tpw new tokens x the G query heads of KV head h.  S^T = K.Q^T and
// O^T += V^T.P^T per 64-key tile, with the keys of a 32-key half permuted
// so that the S^T accumulator layout is the P^T operand layout (lane l holds
// keys 8 (l / 16) .. + 7 of its column).
struct PrefillWave {
    uint32_t l, a, r, x;
    uint32_t i0;                       // first new token of the wave
    half8_t qb[kColBlocks][2];
    uint32_t limit[kColBlocks];        // last key this lane's column may see
    float scale2;
    float m_run[kColBlocks];
    // acc[0..3]: O^T dims 16 db .. 16 db + 15; acc[4] row 0: the softmax
    // denominator, accumulated by the MFMA from a ones row of V^T.
    float4_t acc[5][kColBlocks];
    half8_t ones;
};

__device__ void prefill_wave_init(PrefillWave& w, const kimkv_prefill_item& item, uint32_t h, PrefillShape shape,
                                  uint32_t QH, uint32_t i0)
{
    constexpr uint32_t D = 64;
    w.l = threadIdx.x & 63u;
    w.a = w.l >> 4;
    w.r = w.l & 15u;
    w.x = (w.l >> 2) & 3u;
    w.i0 = i0;
    uint32_t const T0 = item.token_count - item.new_tokens;
    half8_t const zero8 = {};
#pragma unroll
    for (uint32_t cb = 0; cb < kColBlocks; ++cb) {
        uint32_t const i = i0 + cb * shape.tpw + w.r / shape.G;
        uint32_t const q = h * shape.G + w.r % shape.G;
        bool const valid = i < item.new_tokens;
        w.limit[cb] = T0 + (valid ? i : 0);
        w.qb[cb][0] = zero8;
        w.qb[cb][1] = zero8;
        if (valid) {
            const uint16_t* qrow = item.query + (static_cast<uint64_t>(i) * QH + q) * D;
            w.qb[cb][0] = *reinterpret_cast<const half8_t*>(qrow + w.a * 8);
            w.qb[cb][1] = *reinterpret_cast<const half8_t*>(qrow + 32 + w.a * 8);
        }
        w.m_run[cb] = -INFINITY;
#pragma unroll
        for (uint32_t db = 0; db < 5; ++db) w.acc[db][cb] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    w.scale2 = item.attention_scale * kLog2e;
    _Float16 const one = static_cast<_Float16>(w.r == 0 ? 1.0f : 0.0f);
    w.ones = half8_t{one, one, one, one, one, one, one, one};
}

// Keys [t0, t0 + 64) from the staged tile; nvalid = valid keys from t0 on.
// kMasked: some key of the tile is past nvalid or past a column's limit.
template <bool kMasked>
__device__ inline void prefill_wave_step(PrefillWave& w, const KvTile& tile, uint32_t t0, uint32_t nvalid)
{
    // Column block 0's scores are issued first, so its softmax (VALU) runs
    // while block 1's score MFMAs execute, and block 1's softmax while block
    // 0's output MFMAs execute.
    half8_t kop[2][2][2];
#pragma unroll
    for (uint32_t kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (uint32_t e = 0; e < 2; ++e) {
            uint32_t const t = 32 * kb + 8 * w.x + 4 * e + (w.l & 3u);
            kop[kb][e][0] = tile.k[k_unit(t, w.a)];
            kop[kb][e][1] = tile.k[k_unit(t, 4 + w.a)];
        }
    }
    float4_t s[kColBlocks][2][2];
#pragma unroll
    for (uint32_t cb = 0; cb < kColBlocks; ++cb) {
#pragma unroll
        for (uint32_t kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (uint32_t e = 0; e < 2; ++e) {
                float4_t z = {};
                z = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[kb][e][0], w.qb[cb][0], z, 0, 0, 0);
                s[cb][kb][e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[kb][e][1], w.qb[cb][1], z, 0, 0, 0);
            }
        }
    }
    half8_t vop[2][4];
#pragma unroll
    for (uint32_t kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (uint32_t db = 0; db < 4; ++db) vop[kb][db] = tile.v[v_unit(16 * db + w.r, 4 * kb + w.a)];
    }
#pragma unroll
    for (uint32_t cb = 0; cb < kColBlocks; ++cb) {
        // Element i of s[cb][kb][e] is key t0 + 32 kb + 8 a + 4 e + i of this lane's column.  The max is
        // taken on the unscaled dots (scale2 > 0 keeps the order and rounding is monotonic).
        float mx = -INFINITY;
#pragma unroll
        for (uint32_t kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (uint32_t e = 0; e < 2; ++e) {
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i) {
                    if (kMasked) {
                        uint32_t const tt = 32 * kb + 8 * w.a + 4 * e + i;
                        if (!(tt < nvalid && t0 + tt <= w.limit[cb])) s[cb][kb][e][i] = -INFINITY;
                    }
                    mx = fmaxf(mx, s[cb][kb][e][i]);
                }
            }
        }
        // Lazy running max: the reference point moves (and the accumulators
        // are rescaled) only when a score exceeds it by more than 2^8, so
        // p <= 256 stays well inside fp16 and most tiles skip the rescale.
        // The test runs on this lane's 16 keys; only a tile where some lane
        // passes it takes the column max across the four row groups (a
        // column's m stays the same on all of its lanes).  A column whose
        // keys so far are all masked keeps m = -inf.
        bool const over = mx * w.scale2 > w.m_run[cb] + kLazyRescaleLog2;
        if (__builtin_expect(__any(over), 0)) {
            // Not speculated: the reduction and the multiplies run only on tiles that move the reference point.
            __asm__ volatile("" ::: "memory");
            mx = fmaxf(mx, xor16(mx));
            mx = fmaxf(mx, xor32(mx));
            float const m_cand = fmaxf(w.m_run[cb], mx * w.scale2);
            bool const grow = m_cand > w.m_run[cb] + kLazyRescaleLog2;
            float const alpha = grow ? __builtin_amdgcn_exp2f(w.m_run[cb] - m_cand) : 1.0f;
            if (grow) w.m_run[cb] = m_cand;
#pragma unroll
            for (uint32_t db = 0; db < 5; ++db) w.acc[db][cb] *= alpha;
        }
        float const mref = w.m_run[cb];
        bool const empty = kMasked && mref == -INFINITY;
        half8_t pb[2];
#pragma unroll
        for (uint32_t kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (uint32_t e = 0; e < 2; ++e) {
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i) {
                    float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[cb][kb][e][i], w.scale2, -mref));
                    if (kMasked && empty) p = 0.0f;
                    pb[kb][4 * e + i] = static_cast<_Float16>(p);
                }
            }
        }
#pragma unroll
        for (uint32_t kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (uint32_t db = 0; db < 4; ++db) {
                w.acc[db][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop[kb][db], pb[kb], w.acc[db][cb], 0, 0, 0);
            }
            w.acc[4][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w.ones, pb[kb], w.acc[4][cb], 0, 0, 0);
        }
    }
}

__device__ void prefill_wave_store(PrefillWave& w, const kimkv_prefill_item& item, uint32_t h, PrefillShape shape,
                                   uint32_t QH)
{
    constexpr uint32_t D = 64;
#pragma unroll
    for (uint32_t cb = 0; cb < kColBlocks; ++cb) {
        // Row 0 of acc[4] (element 0 on lanes 0..15) is the denominator; the other lanes hold zeros.
        float l_tot = w.acc[4][cb][0] + xor16(w.acc[4][cb][0]);
        l_tot += xor32(l_tot);
        uint32_t const i = w.i0 + cb * shape.tpw + w.r / shape.G;
        if (i >= item.new_tokens) continue;
        uint32_t const q = h * shape.G + w.r % shape.G;
        float const inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        uint16_t* out = item.output + (static_cast<uint64_t>(i) * QH + q) * D;
#pragma unroll
        for (uint32_t db = 0; db < 4; ++db) {
            uint32_t lo = static_cast<uint32_t>(__half_as_ushort(__float2half_rn(w.acc[db][cb][0] * inv)))
                | (static_cast<uint32_t>(__half_as_ushort(__float2half_rn(w.acc[db][cb][1] * inv))) << 16);
            uint32_t hi = static_cast<uint32_t>(__half_as_ushort(__float2half_rn(w.acc[db][cb][2] * inv)))
                | (static_cast<uint32_t>(__half_as_ushort(__float2half_rn(w.acc[db][cb][3] * inv))) << 16);
            *reinterpret_cast<uint2*>(out + db * 16 + 4 * w.a) = make_uint2(lo, hi);
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

// Either order != nullptr (an ordered launch: dispatch index -> XCD-logical
// index -> order entry) or block_prefix != nullptr (head-major blocks, the
// blocks of an item from its last tokens to its first).
__global__ __launch_bounds__(kBlock, 2) void prefill_kernel(PoolView P, const kimkv_prefill_item* items,
                                                            const uint32_t* block_prefix,
                                                            const kimkv_prefill_block* order, uint32_t item_count,
                                                            uint32_t total_blocks, uint32_t QH)
{
    __shared__ HeadGroup groups[kSegmentGroups];
    __shared__ KvTile tiles[2];
    __shared__ GenericScratch scratch[kWaves];
    __shared__ uint32_t s_item;
    __shared__ uint32_t s_generic;
    __shared__ uint32_t s_holes;

    uint32_t const tid = threadIdx.x;
    // Head-major logical order, XCD-contiguous: the blocks of one (item, KV
    // head) run on one XCD and read that head's pages through one L2.
    uint32_t const logical = xcd_logical_index(blockIdx.x, gridDim.x);
    uint32_t block = logical % total_blocks;
    uint32_t h = logical / total_blocks;
    if (tid == 0) {
        s_item = 0xFFFFFFFFu;
        s_generic = 0;
    }
    if (order != nullptr) {
        kimkv_prefill_block const e = order[logical];
        if (tid == 0 && e.item < item_count) s_item = e.item;
        h = e.head;
        block = e.block;
    }
    __syncthreads();
    if (order == nullptr) {
        for (uint32_t k = tid; k < item_count; k += kBlock) {
            if (block_prefix[k] <= block && block < block_prefix[k + 1]) s_item = k;
        }
        __syncthreads();
    }
    uint32_t const it = s_item;
    if (it == 0xFFFFFFFFu) return;
    kimkv_prefill_item const item = items[it];
    uint32_t const H = P.heads;
    uint32_t const D = P.dim;
    if (h >= H || item.new_tokens == 0 || item.new_tokens > item.token_count || item.descriptors == nullptr
        || item.descriptor_count == 0 || item.query == nullptr || item.output == nullptr || item.layer >= P.layers
        || QH == 0 || QH % H != 0 || D > 256) {
        report_fault(P, KIMKV_FAULT_PREFILL_ITEM);
        return;
    }
    PrefillShape const shape = prefill_shape(QH, H, D);
    uint32_t const wave = tid >> 6;
    uint32_t const per_block = prefill_block_tokens(shape);
    // Unordered: the blocks of an item run from its last tokens (most keys) to its first.
    uint32_t const i_block = order != nullptr
        ? block * per_block
        : (block_prefix[it + 1] - 1 - block) * per_block;
    if (i_block >= item.new_tokens) return;
    uint32_t const T0 = item.token_count - item.new_tokens;
    // Keys the whole block needs: [0, T0 + last token of the block].
    uint32_t const last = min(i_block + per_block, item.new_tokens) - 1;
    uint32_t const kend = T0 + last + 1;

    if (shape.mfma) {
        uint32_t const wave_tokens = kColBlocks * shape.tpw;
        uint32_t const i0 = i_block + wave * wave_tokens;
        PrefillWave w;
        prefill_wave_init(w, item, h, shape, QH, i0);
        bool const wave_has_rows = i0 < item.new_tokens;
        // Keys up to the wave's last token (exclusive end) and its first token's limit.
        uint32_t const wave_kend = wave_has_rows ? T0 + min(i0 + wave_tokens, item.new_tokens) : 0;
        uint32_t const wave_full = T0 + i0;   // keys below this need no causal mask
        for (uint32_t s0 = 0; s0 < kend; s0 += kSegmentKeys) {
            uint32_t const s1 = min(s0 + kSegmentKeys, kend);
            uint32_t const ngroups = (s1 - s0 + 7) / 8;
            for (uint32_t g = tid; g < ngroups; g += kBlock) groups[g] = HeadGroup{nullptr, nullptr, 0, 0, 0};
            __syncthreads();
            uint32_t const idx0 = find_descriptor_wave(item.descriptors, item.descriptor_count, s0);
            for (uint32_t j = tid; j <= ngroups && idx0 + j < item.descriptor_count; j += kBlock) {
                add_head_groups(P, item.descriptors[idx0 + j], item.layer, h, s0, s1, item.token_count, groups,
                                &s_generic);
            }
            __syncthreads();
            if (s_generic != 0) break;
            // A group no entry covers (a table with a hole) keeps every tile on the checked loads.
            if (tid == 0) s_holes = 0;
            __syncthreads();
            for (uint32_t g = tid; g < ngroups; g += kBlock) {
                if (groups[g].k == nullptr) s_holes = 1;
            }
            __syncthreads();
            bool const holes = s_holes != 0;
            uint32_t const ntiles = (s1 - s0 + kTileKeys - 1) / kTileKeys;
            // Tile j is computed from tiles[j % 2] while tile j + 1 sits in the
            // other register set and tile j + 2's loads are issued: each tile's
            // loads have two compute phases to land.
            auto compute = [&](const KvTile& tile, uint32_t j) {
                uint32_t const t0 = s0 + j * kTileKeys;
                if (t0 >= wave_kend) return;
                if (t0 + kTileKeys <= s1 && t0 + kTileKeys <= wave_full) {
                    prefill_wave_step<false>(w, tile, t0, s1 - t0);
                } else {
                    prefill_wave_step<true>(w, tile, t0, s1 - t0);
                }
            };
            auto fetch = [&](TileLoad& ld, uint32_t j) {
                uint32_t const nvalid = s1 - s0 - j * kTileKeys;
                if (!holes && nvalid >= kTileKeys) {
                    tile_fetch<true>(ld, groups, j * (kTileKeys / 8), nvalid, tid);
                } else {
                    tile_fetch<false>(ld, groups, j * (kTileKeys / 8), nvalid, tid);
                }
            };
            TileLoad la, lb;
            fetch(la, 0);
            tile_store(tiles[0], la, tid);
            if (ntiles > 1) fetch(lb, 1);
            __syncthreads();
            for (uint32_t j = 0; j < ntiles; j += 2) {
                if (j + 2 < ntiles) fetch(la, j + 2);
                compute(tiles[0], j);
                if (j + 1 < ntiles) tile_store(tiles[1], lb, tid);
                __syncthreads();
                if (j + 1 >= ntiles) break;
                if (j + 3 < ntiles) fetch(lb, j + 3);
                compute(tiles[1], j + 1);
                if (j + 2 < ntiles) tile_store(tiles[0], la, tid);
                __syncthreads();
            }
        }
        if (s_generic == 0) {
            if (wave_has_rows) prefill_wave_store(w, item, h, shape, QH);
            return;
        }
    }
    // Generic path: this wave's new tokens x the G query heads, one row at a time.
    uint32_t const g0 = i_block + wave * (per_block / kWaves);
    uint32_t const g1 = min(g0 + per_block / kWaves, item.new_tokens);
    for (uint32_t i = g0; i < g1; ++i) {
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
    return prefill_block_tokens(prefill_shape(query_heads, storage->layout.kv_heads, storage->layout.head_dim));
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
    if (static_cast<uint64_t>(total_blocks) * storage->layout.kv_heads > 0x7FFFFFFFull) return KIMKV_INVALID_ARGUMENT;
    dim3 const grid(total_blocks * storage->layout.kv_heads);
    void* start = nullptr;
    kernel_timing_begin(TimedKernel::Prefill, native(stream), &start);
    prefill_kernel<<<grid, kBlock, 0, native(stream)>>>(pool_view(*storage), device_items, device_block_prefix,
                                                        nullptr, item_count, total_blocks, query_heads);
    kimkv_status const st = launch_status();
    kernel_timing_end(TimedKernel::Prefill, native(stream), start);
    return st;
}

kimkv_status kimkv_prefill_order(uint32_t kv_heads, uint32_t head_dim, uint32_t query_heads, uint32_t compute_units,
                                 const uint32_t* token_counts, const uint32_t* new_tokens, uint32_t item_count,
                                 kimkv_prefill_block* order, uint32_t capacity, uint32_t* order_count)
{
    if (order_count == nullptr || (item_count != 0 && (token_counts == nullptr || new_tokens == nullptr))
        || query_heads == 0 || kv_heads == 0 || kv_heads > 0xFFFFu || query_heads % kv_heads != 0) {
        return KIMKV_INVALID_ARGUMENT;
    }
    uint32_t const per = prefill_block_tokens(prefill_shape(query_heads, kv_heads, head_dim));
    uint32_t const H = kv_heads;
    struct Unit {
        uint64_t cost;
        kimkv_prefill_block b;
    };
    struct Pair {
        uint64_t cost;
        std::vector<Unit> units;
    };
    // A block's work grows with the keys its last token sees.
    std::vector<Pair> pairs;
    for (uint32_t i = 0; i < item_count; ++i) {
        uint32_t const n = new_tokens[i];
        if (n == 0 || n > token_counts[i]) continue;
        uint32_t const nb = (n + per - 1) / per;
        if (nb > 0xFFFFu) return KIMKV_INVALID_ARGUMENT;
        for (uint32_t h = 0; h < H; ++h) {
            Pair p{0, {}};
            for (uint32_t b = nb; b-- > 0;) {
                uint64_t const keys = static_cast<uint64_t>(token_counts[i]) - n + std::min((b + 1) * per, n);
                Unit u{(keys + 63) / 64 + 1, kimkv_prefill_block{i, static_cast<uint16_t>(h), static_cast<uint16_t>(b)}};
                p.cost += u.cost;
                p.units.push_back(u);
            }
            pairs.push_back(std::move(p));
        }
    }
    // Whole (item, head) pairs to XCDs, heaviest first onto the least loaded;
    // with fewer pairs than XCDs the blocks themselves are spread.
    std::vector<std::vector<Unit>> xcd(kXcds);
    std::vector<uint64_t> load(kXcds, 0);
    auto least = [&] {
        uint32_t x = 0;
        for (uint32_t k = 1; k < kXcds; ++k) {
            if (load[k] < load[x] || (load[k] == load[x] && xcd[k].size() < xcd[x].size())) x = k;
        }
        return x;
    };
    if (pairs.size() >= kXcds) {
        std::stable_sort(pairs.begin(), pairs.end(), [](Pair const& a, Pair const& b) { return a.cost > b.cost; });
        for (Pair& p : pairs) {
            uint32_t const x = least();
            load[x] += p.cost;
            xcd[x].insert(xcd[x].end(), p.units.begin(), p.units.end());
        }
    } else {
        std::vector<Unit> all;
        for (Pair& p : pairs) all.insert(all.end(), p.units.begin(), p.units.end());
        std::stable_sort(all.begin(), all.end(), [](Unit const& a, Unit const& b) { return a.cost > b.cost; });
        for (Unit const& u : all) {
            uint32_t const x = least();
            load[x] += u.cost;
            xcd[x].push_back(u);
        }
    }
    // Inside an XCD: heaviest first; when every block of the XCD is resident
    // at once (two per compute unit), slot k and slot k + CUs share a compute
    // unit, so the second half is reversed to pair heavy with light.
    uint32_t const cus = compute_units >= kXcds ? compute_units / kXcds : 32u;
    size_t len = 0;
    for (auto& list : xcd) {
        std::stable_sort(list.begin(), list.end(), [](Unit const& a, Unit const& b) { return a.cost > b.cost; });
        size_t const m = list.size();
        if (m > cus && m <= 2 * static_cast<size_t>(cus)) std::reverse(list.begin() + cus, list.end());
        len = std::max(len, m);
    }
    uint64_t const total = len * kXcds;
    if (total > 0x7FFFFFFFull) return KIMKV_INVALID_ARGUMENT;
    *order_count = static_cast<uint32_t>(total);
    if (capacity < total || (total != 0 && order == nullptr)) return KIMKV_INVALID_ARGUMENT;
    // XCD x owns logical entries [x * len, (x + 1) * len) (xcd_logical_index
    // with a multiple of 8 entries); short lists end in idle slots.
    for (uint32_t x = 0; x < kXcds; ++x) {
        for (size_t k = 0; k < len; ++k) {
            order[x * len + k] = k < xcd[x].size() ? xcd[x][k].b : kimkv_prefill_block{0xFFFFFFFFu, 0, 0};
        }
    }
    return KIMKV_OK;
}

kimkv_status kimkv_paged_prefill_ordered(const kimkv_storage* storage, const kimkv_prefill_item* device_items,
                                         uint32_t item_count, const kimkv_prefill_block* device_order,
                                         uint32_t order_count, uint32_t query_heads, kimkv_stream_t stream)
{
    if (storage == nullptr || device_items == nullptr || device_order == nullptr || query_heads == 0
        || storage->layout.kv_heads == 0 || query_heads % storage->layout.kv_heads != 0
        || storage->layout.head_dim > 256 || order_count > 0x7FFFFFFFu) {
        return KIMKV_INVALID_ARGUMENT;
    }
    if (order_count == 0 || item_count == 0) return KIMKV_OK;
    void* start = nullptr;
    kernel_timing_begin(TimedKernel::Prefill, native(stream), &start);
    prefill_kernel<<<order_count, kBlock, 0, native(stream)>>>(pool_view(*storage), device_items, nullptr,
                                                               device_order, item_count, 1u, query_heads);
    kimkv_status const st = launch_status();
    kernel_timing_end(TimedKernel::Prefill, native(stream), start);
    return st;
}

}  // extern "C"
