// decode_kernels.hip -- fused split-K GQA paged decode attention for gfx950.
//
// Replaces pagedAttentionScores*/pagedAttentionOutput* (scores then output,
// src/cuda/attention/paged_decode_kernels.cu:132-474) with one pass over the
// KV pages.  Work unit: a workgroup per (lane, chunk of tokens, group of four
// kv heads); wave w owns kv head h and that head's query group.
//
// Fast path (head_dim 64, group <= 16, page-aligned table): per 64-token tile
//   S^T[token][q] = K[token][:] . Q[q][:]   -> 4 x 2 MFMA 16x16x32 f16
//   online softmax (base 2) on the 16 scores each lane holds
//   O^T[d][q]    += V^T[d][token] . P[q][token] -> 2 x 4 x 2 MFMA 16x16x32 f16
//                   (P split into fp16 hi and lo parts: ~fp32 weights)
// K rows and V^T rows (V is stored transposed in the page) are read with
// 16-byte loads straight into MFMA operand registers; the token order inside
// each 32-token k-block is permuted so that the score layout MFMA produces is
// exactly the P operand layout the second MFMA consumes (no shuffles).
// Lanes with more than one chunk write (o, m, l) partials to the lane
// workspace; combine_kernel merges them.
#include <hip/hip_runtime.h>

#include <cmath>
#include <mutex>
#include <type_traits>

#include "attention_common.h"
#include "device_common.h"
#include "runtime_internal.h"

namespace kimkv {
namespace {

constexpr unsigned kBlock = 256;          // 4 waves
constexpr unsigned kHeadsPerBlock = 4;
constexpr unsigned kMinChunk = 256;
constexpr unsigned kWholeLaneMax = 1024;   // tokens: longest lane a small batch keeps whole
// Softmax weights of the fast path are 2^(s - m + kWeightShift): the largest
// is 2^15 (fp16 max 65504), and weights down to 2^-29 of the largest stay
// fp16 normal numbers.  o and l carry the same factor, so it cancels in the
// output and in every merge of partials.
constexpr float kWeightShift = 15.0f;

// ---------------------------------------------------------------------------
// Fast path for one wave: kv head h, head_dim 64, group <= 16.
// ---------------------------------------------------------------------------
// Online-softmax state of one wave over its tokens: lane (a, r) holds
// O^T[d][r] for d = 16 db + 4 a + i in acc[db][i], and the running max m and
// denominator l of query column r (the same in every lane group a).
struct WavePartial {
    float4_t acc[4];
    float m;
    float l;
};

// A K or V^T operand load: non-temporal (streamed past the caches) for long
// chunks and large launches, where every byte is read once and the
// streaming hint keeps HBM busier (7.1 vs 6.2 TB/s in a read probe; the
// 128-lane x 32k launch is 0.656 instead of 0.640 ms without it); cached for
// short chunks in small, latency-bound launches (the 32-lane shared-prefix
// layer: 24.9 instead of 26.4 us).
template <bool kStream>
__device__ __attribute__((always_inline)) inline half8_t load_kv(const uint16_t* p)
{
    return kStream ? load_half8_stream(p) : load_half8(p);
}

// A score times the folded scale (attention scale * log2 e), rounded on its
// own: kept out of FMA contraction with the exponent's subtraction so that
// full steps and tail steps (a chunk's last step, or the step that reads a
// write job's new token) give the same bits for the same token.
__device__ inline float scaled_score(float s, float scale2)
{
#pragma clang fp contract(off)
    return s * scale2;
}

// The lane's new token as one kv head reads it in a launch that also writes
// it: its K and V rows ([D] each) come from the write job's source, not from
// the page (whose store is issued at the end of the launch).  t = absolute
// token index, kNoToken when the chunk reads no new token.
constexpr uint32_t kNoToken = 0xFFFFFFFFu;
struct NewTokenRows {
    const uint16_t* key;
    const uint16_t* value;
    uint32_t t;
};

// Tokens [c0, c1) of kv head h; the group table starts at token g0 (c0 - g0
// is a multiple of 64).  When nt.t == c1 - 1 the last token's K and V come
// from nt's rows (its page group may hold anything at that position).
template <bool kStream>
__device__ WavePartial decode_wave_d64(const GroupEntry* groups, const GroupResolver& res,
                                       const kimkv_decode_item& item, uint32_t h, uint32_t G, uint32_t g0,
                                       uint32_t c0, uint32_t c1, NewTokenRows const& nt)
{
    constexpr uint32_t D = 64;
    uint32_t const l = threadIdx.x & 63u;
    uint32_t const a = l >> 4;            // lane group
    uint32_t const r = l & 15u;           // row/column inside a 16-wide MFMA tile
    uint32_t const x = (l >> 2) & 3u;     // K-operand row group
    uint32_t const q = h * G + r;
    bool const qvalid = r < G;
    // The new token is always read in the tail variant of the last step.
    bool const has_new = nt.t != kNoToken && nt.t + 1 == c1;
    uint32_t const new_t = has_new ? nt.t : kNoToken;

    half8_t qb0 = {};
    half8_t qb1 = {};
    if (qvalid) {
        qb0 = load_half8(item.query + static_cast<uint64_t>(q) * D + a * 8);
        qb1 = load_half8(item.query + static_cast<uint64_t>(q) * D + 32 + a * 8);
    }
    float const scale2 = item.attention_scale * kLog2e;
    float m_run = -INFINITY;
    float l_part = 0.0f;
    float4_t acc[4] = {};
    half8_t const zero8 = {};

    // One 64-token step is a load phase (K rows and V^T rows of the step into
    // registers) and a compute phase; the next step's loads are issued before
    // the current step's compute (two register buffers), so each wave keeps
    // up to two steps of K/V in flight and the compute hides under them.  The
    // tail variants mask tokens past the chunk end; full steps skip every
    // per-token compare and load unconditionally (the caller guarantees every
    // group of the chunk is mapped), so the waits before a compute cover
    // exactly the older buffer's loads.
    struct Ops {
        half8_t k[2][2][2];
        half8_t v[2][4];
    };
    auto load = [&](Ops& o, uint32_t t0, auto tail) {
        constexpr bool kTail = decltype(tail)::value;
        uint32_t const tg = (t0 - g0) >> 3;
        uint32_t const nvalid = c1 - t0;
#pragma unroll
        for (uint32_t kb = 0; kb < 2; ++kb) {
            GroupEntry const gk = groups[tg + 4 * kb + x];
#pragma unroll
            for (uint32_t e = 0; e < 2; ++e) {
                uint32_t const tt = 32 * kb + 8 * x + 4 * e + (l & 3u);
                if (kTail && t0 + tt == new_t) {
                    // The new token's K row: dims [8a, 8a+8) and [32+8a, 40+8a) of the source.
                    o.k[kb][e][0] = load_half8(nt.key + a * 8);
                    o.k[kb][e][1] = load_half8(nt.key + 32 + a * 8);
                } else if (!kTail || (tt < nvalid && gk.page != kUnmappedGroup)) {
                    // K column blocks of 32 dims: dims [8a, 8a+8) and [32+8a, 40+8a).
                    const uint16_t* row = res.block(gk) + static_cast<uint64_t>(gk.pt0 + 4 * e + (l & 3u)) * 32
                        + a * 8;
                    o.k[kb][e][0] = load_kv<kStream>(row);
                    o.k[kb][e][1] = load_kv<kStream>(row + static_cast<uint64_t>(gk.cap) * 32);
                } else {
                    o.k[kb][e][0] = zero8;
                    o.k[kb][e][1] = zero8;
                }
            }
            GroupEntry const gv = groups[tg + 4 * kb + a];
            uint32_t const vt0 = 32 * kb + 8 * a;
            if (!kTail || (vt0 < nvalid && gv.page != kUnmappedGroup)) {
                // V^T column block of vw tokens holding this 8-token group; row d = 16 db + r.
                uint32_t const vw = v_width(gv.cap);
                const uint16_t* vt = res.block(gv) + v_offset(gv.cap, D, gv.pt0, r);
#pragma unroll
                for (uint32_t db = 0; db < 4; ++db) {
                    o.v[kb][db] = load_kv<kStream>(vt + static_cast<uint64_t>(db * 16) * vw);
                }
            } else {
#pragma unroll
                for (uint32_t db = 0; db < 4; ++db) o.v[kb][db] = zero8;
            }
        }
    };
    auto compute = [&](Ops& o, uint32_t t0, auto tail) {
        constexpr bool kTail = decltype(tail)::value;
        uint32_t const nvalid = c1 - t0;
        if (kTail) {
            // Tokens past the chunk end may hold stale data: zero their V.
#pragma unroll
            for (uint32_t kb = 0; kb < 2; ++kb) {
                uint32_t const vt0 = 32 * kb + 8 * a;
                if (vt0 < nvalid && vt0 + 8 > nvalid) {
                    uint32_t const keep = nvalid - vt0;
#pragma unroll
                    for (uint32_t db = 0; db < 4; ++db) {
#pragma unroll
                        for (uint32_t j = 0; j < 8; ++j) {
                            if (j >= keep) o.v[kb][db][j] = static_cast<_Float16>(0.0f);
                        }
                    }
                }
            }
        }

        // ---- scores ----
        float4_t s[2][2];
#pragma unroll
        for (uint32_t kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (uint32_t e = 0; e < 2; ++e) {
                float4_t z = {};
                z = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.k[kb][e][0], qb0, z, 0, 0, 0);
                s[kb][e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.k[kb][e][1], qb1, z, 0, 0, 0);
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (uint32_t kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (uint32_t e = 0; e < 2; ++e) {
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i) {
                    uint32_t const tt = 32 * kb + 8 * a + 4 * e + i;
                    float const v = !kTail || tt < nvalid ? scaled_score(s[kb][e][i], scale2) : -INFINITY;
                    s[kb][e][i] = v;
                    mx = fmaxf(mx, v);
                }
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        float const m_new = fmaxf(m_run, mx);
        float const alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;

        // Weights p = 2^(s - m + kWeightShift) <= 2^15 go to the MFMA as two
        // fp16 parts, p = hi + lo (hi = fp16(p), lo = fp16(p - hi)), so the
        // products with V carry ~22 significant bits, like the fp32 weights
        // of the reference, and the denominator sums the same p.  The shift
        // keeps small weights in fp16's normal range; it cancels in o / l.
        float const m_ref = m_new - kWeightShift;
        half8_t pb[2];
        half8_t pl[2];
        float psum = 0.0f;
#pragma unroll
        for (uint32_t kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (uint32_t e = 0; e < 2; ++e) {
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i) {
                    float const p = __builtin_amdgcn_exp2f(s[kb][e][i] - m_ref);
                    _Float16 const hi = static_cast<_Float16>(p);
                    psum += p;
                    pb[kb][4 * e + i] = hi;
                    pl[kb][4 * e + i] = static_cast<_Float16>(p - static_cast<float>(hi));
                }
            }
        }
        l_part = l_part * alpha + psum;
#pragma unroll
        for (uint32_t db = 0; db < 4; ++db) acc[db] *= alpha;

        // ---- O^T += V^T . (P_hi + P_lo)^T ----
#pragma unroll
        for (uint32_t kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (uint32_t db = 0; db < 4; ++db) {
                acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.v[kb][db], pb[kb], acc[db], 0, 0, 0);
                acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.v[kb][db], pl[kb], acc[db], 0, 0, 0);
            }
        }
    };
    Ops buf_a;
    Ops buf_b;
    std::false_type const full{};
    uint32_t const nfull = (has_new ? c1 - c0 - 1 : c1 - c0) >> 6;
    if (nfull > 0) {
        // At the top of each round buf_a holds step s - 1 in flight; the body
        // has no bounds test, so no load in it is conditional.
        load(buf_a, c0, full);
        uint32_t s = 1;
        for (; s + 1 < nfull; s += 2) {
            load(buf_b, c0 + 64 * s, full);
            compute(buf_a, c0, full);
            load(buf_a, c0 + 64 * (s + 1), full);
            compute(buf_b, c0, full);
        }
        if (s < nfull) {
            load(buf_b, c0 + 64 * s, full);
            compute(buf_a, c0, full);
            compute(buf_b, c0, full);
        } else {
            compute(buf_a, c0, full);
        }
    }
    if (c0 + 64 * nfull < c1) {
        uint32_t const t0 = c0 + 64 * nfull;
        load(buf_a, t0, std::true_type{});
        if (has_new) {
            // V^T rows d = 16 db + r of the new token's 8-token group: element
            // j of lane group a (tokens [32 kb + 8 a, +8) of the step) is the
            // new token for one (kb, a).
#pragma unroll
            for (uint32_t kb = 0; kb < 2; ++kb) {
                uint32_t const j = new_t - t0 - (32 * kb + 8 * a);
                if (j < 8) {
#pragma unroll
                    for (uint32_t db = 0; db < 4; ++db) {
                        buf_a.v[kb][db][j] = __builtin_bit_cast(_Float16, nt.value[16 * db + r]);
                    }
                }
            }
        }
        compute(buf_a, t0, std::true_type{});
    }

    float l_tot = l_part + __shfl_xor(l_part, 16);
    l_tot += __shfl_xor(l_tot, 32);
    WavePartial out;
#pragma unroll
    for (uint32_t db = 0; db < 4; ++db) out.acc[db] = acc[db];
    out.m = m_run;
    out.l = l_tot;
    return out;
}

// Writes dims [d0, d0 + 4) of query head q: the fp16 output when the lane
// has one chunk, else the chunk's (o, m, l) partial for combine_kernel (m and
// l by the one caller per row that passes write_ml).
__device__ inline void store_partial(const kimkv_decode_item& item, uint32_t QH, uint32_t q, uint32_t chunk_index,
                                     bool single_chunk, float4_t o, uint32_t d0, float m, float l, bool write_ml)
{
    constexpr uint32_t D = 64;
    if (single_chunk) {
        float const inv = 1.0f / l;
        uint16_t* out = item.output + static_cast<uint64_t>(q) * D + d0;
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) out[i] = __half_as_ushort(__float2half_rn(o[i] * inv));
    } else {
        float* ws = item.workspace + (static_cast<uint64_t>(chunk_index) * QH + q) * (D + 2);
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) ws[d0 + i] = o[i];
        if (write_ml) {
            ws[D] = m;
            ws[D + 1] = l;
        }
    }
}

// ---------------------------------------------------------------------------
// Generic path for one wave: any head_dim <= 256, any group size, any table.
// One query head at a time; lanes own tokens for scores and dims for output.
// ---------------------------------------------------------------------------
struct WaveTokens {
    float p[64];
    const uint16_t* head[64];   // (layer, head) block of the token's page; the V row when cap == 0
    uint32_t cap[64];
    uint32_t pt[64];
};

// A lane's single-token write job (kimkv_paged_decode_write_batch) as the
// decode reads the pages: positions of the destination page that the job
// writes are read from where the job takes them -- [0, cow_tokens) from the
// copy-on-write source page, dst_token from the job's rows -- never from the
// destination page.  So no read of the launch depends on the job's stores,
// and the workgroups that make them issue them last.  `active` is false when
// the lane has no job or the job is invalid.
struct JobView {
    bool active;
    uint32_t dst_tag;        // GroupEntry::page form of the destination page
    uint32_t cow_tag;        // and of the copy-on-write source
    uint32_t dst_kind;
    uint32_t dst_slot;
    uint32_t dst_token;
    uint32_t cow_kind;
    uint32_t cow_slot;
    uint32_t cow_tokens;
    uint32_t cow_cap;
    const uint16_t* key;     // the new token's rows [H][D]
    const uint16_t* value;
};

// A job kimkv_paged_decode_write_batch can apply to `layer`: one token of one
// layer into a page of this storage, an optional copy-on-write source that
// holds the copied positions.
__device__ inline bool write_job_valid(const PoolView& P, const kimkv_append_job& job, uint32_t layer)
{
    uint32_t const dcap = pool_tokens(P, job.dst_kind);
    if (page_base(P, job.dst_kind, job.dst_slot, dcap) == nullptr || job.token_count != 1 || job.layer_count != 1
        || job.layer_begin != layer || layer >= P.layers || job.dst_token >= dcap || job.src_key == nullptr
        || job.src_value == nullptr) {
        return false;
    }
    if (job.cow_tokens != 0) {
        uint32_t const scap = pool_tokens(P, job.cow_kind);
        if (page_base(P, job.cow_kind, job.cow_slot, scap) == nullptr || job.cow_tokens > scap
            || job.cow_tokens > job.dst_token) {
            return false;
        }
    }
    return true;
}

__device__ inline uint32_t group_tag(uint32_t kind, uint32_t slot)
{
    return kind == KIMKV_PAGE_EXTENT ? slot | kExtentPage : slot;
}

__device__ inline JobView job_view(const PoolView& P, const kimkv_append_job& job, bool valid)
{
    JobView v{};
    v.active = valid;
    if (!valid) return v;
    v.dst_kind = job.dst_kind;
    v.dst_slot = job.dst_slot;
    v.dst_token = job.dst_token;
    v.dst_tag = group_tag(job.dst_kind, job.dst_slot);
    v.cow_tokens = job.cow_tokens;
    v.cow_kind = job.cow_kind;
    v.cow_slot = job.cow_slot;
    v.cow_tag = group_tag(job.cow_kind, job.cow_slot);
    v.cow_cap = job.cow_tokens != 0 ? pool_tokens(P, job.cow_kind) : 0;
    v.key = job.src_key;
    v.value = job.src_value;
    return v;
}

__device__ void decode_wave_generic(const PoolView& P, const kimkv_decode_item& item, uint32_t h,
                                    uint32_t G, uint32_t QH, uint32_t c0, uint32_t c1,
                                    uint32_t chunk_index, bool single_chunk, WaveTokens* tokens, JobView const& jv)
{
    uint32_t const lane = threadIdx.x & 63u;
    uint32_t const D = P.dim;
    uint32_t const layer = item.layer;
    float const scale2 = item.attention_scale * kLog2e;
    for (uint32_t j = 0; j < G; ++j) {
        uint32_t const q = h * G + j;
        const uint16_t* qv = item.query + static_cast<uint64_t>(q) * D;
        float m_run = -INFINITY;
        float l_run = 0.0f;
        float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (uint32_t t0 = c0; t0 < c1; t0 += 64) {
            uint32_t const t = t0 + lane;
            bool const valid = t < c1;
            uint32_t idx = find_descriptor_wave(item.descriptors, item.descriptor_count, t0);
            const uint16_t* page = nullptr;
            uint32_t cap = 0;
            uint32_t pt = 0;
            if (valid) {
                while (idx + 1 < item.descriptor_count
                       && item.descriptors[idx + 1].logical_token_begin <= t) {
                    ++idx;
                }
                kimkv_block_desc const e = item.descriptors[idx];
                if (t >= e.logical_token_begin && t < e.logical_token_begin + e.valid_tokens
                    && e.valid_tokens <= e.page_token_capacity) {
                    page = page_base(P, e.kind, e.slot, e.page_token_capacity);
                    cap = e.page_token_capacity;
                    pt = t - e.logical_token_begin;
                }
            }
            float s = -INFINITY;
            const uint16_t* hb = nullptr;
            if (page != nullptr) {
                hb = page + head_block(P, cap, layer, h);
                const uint16_t* krow = nullptr;   // contiguous K row when the job supplies the token
                if (jv.active && page == page_base(P, jv.dst_kind, jv.dst_slot, pool_tokens(P, jv.dst_kind))) {
                    if (pt == jv.dst_token) {
                        krow = jv.key + static_cast<uint64_t>(h) * D;
                        hb = jv.value + static_cast<uint64_t>(h) * D;
                        cap = 0;
                    } else if (pt < jv.cow_tokens) {
                        hb = page_base(P, jv.cow_kind, jv.cow_slot, jv.cow_cap) + head_block(P, jv.cow_cap, layer, h);
                        cap = jv.cow_cap;
                    }
                }
                float dot = 0.0f;
                for (uint32_t d = 0; d < D; ++d) {
                    uint16_t const kc = krow != nullptr ? krow[d] : hb[k_offset(cap, D, pt, d)];
                    dot += __half2float(__ushort_as_half(qv[d])) * __half2float(__ushort_as_half(kc));
                }
                s = dot * scale2;
            }
            float const m_new = fmaxf(m_run, wave_max(s));
            float const alpha = m_new == -INFINITY ? 1.0f : exp2f(m_run - m_new);
            // Same weight shift as the fast path: partials of one lane may
            // come from both paths and are merged as they are.
            float const p = (page != nullptr && m_new != -INFINITY) ? exp2f(s - m_new + kWeightShift) : 0.0f;
            l_run = l_run * alpha + wave_sum(p);
            m_run = m_new;
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] *= alpha;
            tokens->p[lane] = p;
            tokens->head[lane] = hb;
            tokens->cap[lane] = cap;
            tokens->pt[lane] = pt;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            uint32_t const nt = min(64u, c1 - t0);
            for (uint32_t tt = 0; tt < nt; ++tt) {
                float const pp = tokens->p[tt];
                const uint16_t* vb = tokens->head[tt];
                uint32_t const vc = tokens->cap[tt];
                uint32_t const vp = tokens->pt[tt];
                if (vb == nullptr || pp == 0.0f) continue;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    uint32_t const d = lane + 64u * k;
                    if (d < D) {
                        uint16_t const vv = vc == 0 ? vb[d] : vb[v_offset(vc, D, vp, d)];
                        o[k] += pp * __half2float(__ushort_as_half(vv));
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        if (single_chunk) {
            float const inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint32_t const d = lane + 64u * k;
                if (d < D) {
                    item.output[static_cast<uint64_t>(q) * D + d] = __half_as_ushort(__float2half_rn(o[k] * inv));
                }
            }
        } else {
            float* ws = item.workspace + (static_cast<uint64_t>(chunk_index) * QH + q) * (D + 2);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint32_t const d = lane + 64u * k;
                if (d < D) ws[d] = o[k];
            }
            if (lane == 0) {
                ws[D] = m_run;
                ws[D + 1] = l_run;
            }
        }
    }
}

// The per-lane conditions decode_kernel checks before touching a lane with
// tokens (the merge skips the same lanes, so a rejected lane's output stays
// unwritten).  `merged`: the launch runs the split-K merge (its chunk count
// exceeds its lane count); without it a lane of several chunks would never
// get its output.
__device__ inline bool decode_item_valid(const PoolView& P, const kimkv_decode_item& item, uint32_t QH,
                                         uint32_t nchunks, bool merged)
{
    return item.token_count != 0 && item.descriptors != nullptr && item.descriptor_count != 0
        && item.query != nullptr && item.output != nullptr && item.layer < P.layers && QH != 0
        && QH % P.heads == 0 && P.dim <= 256 && (nchunks <= 1 || (item.workspace != nullptr && merged));
}

// LDS of a decode workgroup: the chunk's group table (also the buffer the
// head-split merge uses), the per-wave token records of the generic path and
// the lane's write job, kept for the stores at the workgroup's end (the
// caller's job array may live in host memory, a round trip away).
struct DecodeLds {
    __attribute__((aligned(16))) GroupEntry groups[kMaxGroups];
    WaveTokens wave_tokens[kHeadsPerBlock];
    kimkv_append_job job;
    uint32_t idx0;
    uint32_t dok;
    uint32_t generic;
    uint32_t new_ok;   // the chunk reads the write job's new token as its last token
};

// Builds the group table of tokens [c0, c1) of `item` (c0 a multiple of 8)
// and returns whether the fast path applies (head_dim 64, group <= 16, every
// 8-token group mapped and aligned).  With an active write job, groups of
// its destination page below the copied count are read from the
// copy-on-write source page instead, and lds.new_ok says whether the chunk's
// last token is the job's new token (read from the job's rows by the fast
// path); a table the fast path cannot read that way (the destination
// position of the new token read as another token, a group mixing copied
// and kept positions) goes to the generic path, which applies the same rule
// per token.  Called by every thread of the block.
__device__ bool build_chunk_table(const PoolView& P, const kimkv_decode_item& item, uint32_t QH, uint32_t c0,
                                  uint32_t c1, DecodeLds& lds, JobView const& jv)
{
    uint32_t const tid = threadIdx.x;
    uint32_t const T = item.token_count;
    uint32_t const ngroups = (c1 - c0 + 7) / 8;
    if (tid == 0) {
        lds.generic = 0;
        lds.new_ok = 0;
    }
    for (uint32_t g = tid; g < ngroups; g += kBlock) {
        lds.groups[g] = GroupEntry{kUnmappedGroup, 0, 0};
    }
    __syncthreads();

    // First descriptor of the chunk: an entry holds at most 64 tokens, so the
    // one holding c0 has index >= c0 / 64, and equals it when the table is all
    // extents up to c0.  Build the group table from that guess; the thread
    // reading the guessed entry checks that it holds c0.
    uint32_t const dguess = min(c0 / 64u, item.descriptor_count - 1);
    for (uint32_t j = tid; j <= ngroups && dguess + j < item.descriptor_count; j += kBlock) {
        kimkv_block_desc const e = item.descriptors[dguess + j];
        if (j == 0) lds.dok = e.logical_token_begin <= c0 && c0 - e.logical_token_begin < e.valid_tokens ? 1u : 0u;
        add_groups(P, e, c0, c1, T, lds.groups, &lds.generic);
    }
    __syncthreads();
    if (lds.dok == 0) {
        for (uint32_t g = tid; g < ngroups; g += kBlock) {
            lds.groups[g] = GroupEntry{kUnmappedGroup, 0, 0};
        }
        if (tid < 64) {
            uint32_t const idx0 = find_descriptor_wave(item.descriptors, item.descriptor_count, c0);
            if (tid == 0) lds.idx0 = idx0;
        }
        __syncthreads();
        uint32_t const idx0 = lds.idx0;
        for (uint32_t j = tid; j <= ngroups && idx0 + j < item.descriptor_count; j += kBlock) {
            add_groups(P, item.descriptors[idx0 + j], c0, c1, T, lds.groups, &lds.generic);
        }
        __syncthreads();
    }

    // The fast path loads full steps without per-group checks: a chunk with
    // an unmapped 8-token group goes to the generic path, which skips
    // unmapped tokens.
    bool generic = false;
    for (uint32_t g = tid; g < ngroups; g += kBlock) {
        GroupEntry const e = lds.groups[g];
        generic |= e.page == kUnmappedGroup;
        if (!jv.active || e.page != jv.dst_tag) continue;
        uint32_t const rel = jv.dst_token - e.pt0;   // the new token's place in the group, if < 8
        if (rel < 8u) {
            if (c0 + 8 * g + rel == T - 1) {
                lds.new_ok = 1;
            } else {
                generic = true;
            }
        }
        if (jv.cow_tokens != 0 && e.pt0 < jv.cow_tokens) {
            // Positions past the copied ones are the new token or past it
            // (tokens >= T, masked) when cow_tokens == dst_token.
            if ((e.pt0 + 8u <= jv.cow_tokens || jv.cow_tokens == jv.dst_token) && (jv.cow_cap & 7u) == 0) {
                lds.groups[g] = GroupEntry{jv.cow_tag, e.pt0, static_cast<uint16_t>(jv.cow_cap)};
            } else {
                generic = true;
            }
        }
    }
    if (generic) lds.generic = 1;
    __syncthreads();
    uint32_t const G = QH / P.heads;
    return P.dim == 64 && G <= 16 && lds.generic == 0;
}

// A kRecords launch's cache of chunk group tables (optional): the table a
// chunk's workgroup builds from its lane's descriptors is the same for every
// layer of a token step, so the first launch of the step stores it and later
// launches copy it into LDS instead of reading the descriptors -- in the
// same round trip as the lane record, where building it waits for that
// record.  Per chunk: a 16-byte header, then `stride` 8-byte group entries.
// A header whose tag is not the launch's (another step, or never written)
// makes the workgroup build the table, and the chunk's first workgroup
// stores it with the launch's tag and id.  A header stored by the same
// launch is not trusted either: in the head-split mode a chunk has one
// workgroup per kv head, and nothing orders one workgroup's entry stores
// before another's reads within a launch (they may sit on different XCDs),
// while the end of a launch makes its stores visible to the next one.
struct TableCacheHeader {
    uint32_t tag;
    uint32_t launch;    // id of the launch that stored it
    uint32_t ngroups;
    uint32_t flags;     // bit 0: generic path, bit 1: new token readable
};
static_assert(sizeof(TableCacheHeader) == 16 && sizeof(GroupEntry) == 8, "cache layout");

struct TableCache {
    unsigned char* base;   // nullptr: no cache
    uint32_t stride;       // group entries per chunk (chunk_tokens / 8)
    uint32_t tag;          // nonzero
    uint32_t launch;       // this launch's id: nonzero, unique among recent launches
};
// Entries one thread prefetches: chunks of up to 4096 tokens.
constexpr uint32_t kTableCachePerThread = 2;
constexpr uint32_t kTableCacheMaxChunk = kTableCachePerThread * kBlock * 8;

__host__ __device__ inline uint64_t table_cache_chunk_bytes(uint32_t stride)
{
    return sizeof(TableCacheHeader) + static_cast<uint64_t>(stride) * sizeof(GroupEntry);
}

// build_chunk_table for a kRecords launch with a table cache (see
// TableCache): when the header this workgroup loaded with its lane record
// carries the launch's tag, another launch's id and the chunk's group count,
// the entries it copied into lds.groups are the table; otherwise the table
// is built from the descriptors, and the chunk's first workgroup (blockIdx.y
// 0) stores it with the launch's tag and id.  Called by every thread of the
// block.
__device__ inline bool chunk_table_cached(const PoolView& P, const kimkv_decode_item& item, uint32_t QH, uint32_t c0,
                                          uint32_t c1, DecodeLds& lds, JobView const& jv, TableCache const& cache,
                                          uint32_t chunk_id, TableCacheHeader const& s_hdr)
{
    uint32_t const ngroups = (c1 - c0 + 7) / 8;
    if (cache.base == nullptr || ngroups > cache.stride) return build_chunk_table(P, item, QH, c0, c1, lds, jv);
    __syncthreads();   // the header and entries copied into LDS
    uint32_t const G = QH / P.heads;
    if (s_hdr.tag == cache.tag && s_hdr.launch != cache.launch && s_hdr.ngroups == ngroups) {
        if (threadIdx.x == 0) {
            lds.generic = s_hdr.flags & 1u;
            lds.new_ok = (s_hdr.flags >> 1) & 1u;
        }
        __syncthreads();
        return P.dim == 64 && G <= 16 && lds.generic == 0;
    }
    __syncthreads();   // every thread has read the header before the table is rebuilt
    bool const fast = build_chunk_table(P, item, QH, c0, c1, lds, jv);
    if (blockIdx.y == 0) {
        unsigned char* c = cache.base + table_cache_chunk_bytes(cache.stride) * chunk_id;
        for (uint32_t g = threadIdx.x; g < ngroups; g += kBlock) {
            reinterpret_cast<GroupEntry*>(c + sizeof(TableCacheHeader))[g] = lds.groups[g];
        }
        if (threadIdx.x == 0) {
            uint32_t const flags = (lds.generic != 0 ? 1u : 0u) | (lds.new_ok != 0 ? 2u : 0u);
            *reinterpret_cast<TableCacheHeader*>(c) = TableCacheHeader{cache.tag, cache.launch, ngroups, flags};
        }
    }
    return fast;
}

// One (lane, kv head, chunk) by the whole workgroup: tokens [c0, c1) cut
// into four 64-token-aligned quarters, one per wave, the four online-softmax
// states merged through LDS, then the output (single chunk) or the chunk's
// partial written.  Called by every thread of the block after
// build_chunk_table; ends with the merge buffer still in use (callers that
// reuse the LDS synchronize first).
// The new-token rows kv head h of a fast-path chunk reads (kNoToken when the
// chunk's last token is not the write job's new token).
__device__ inline NewTokenRows new_token_rows(const DecodeLds& lds, JobView const& jv, uint32_t T, uint32_t h,
                                              uint32_t D)
{
    if (lds.new_ok == 0) return NewTokenRows{nullptr, nullptr, kNoToken};
    return NewTokenRows{jv.key + static_cast<uint64_t>(h) * D, jv.value + static_cast<uint64_t>(h) * D, T - 1};
}

template <bool kStream>
__device__ void decode_head_split_chunk(const PoolView& P, const kimkv_decode_item& item, uint32_t h, uint32_t QH,
                                        uint32_t c0, uint32_t c1, uint32_t chunk_index, bool single, bool fast,
                                        DecodeLds& lds, JobView const& jv)
{
    uint32_t const tid = threadIdx.x;
    uint32_t const wave = tid >> 6;
    uint32_t const G = QH / P.heads;
    if (!fast) {
        if (wave == 0) {
            decode_wave_generic(P, item, h, G, QH, c0, c1, chunk_index, single, &lds.wave_tokens[0], jv);
        }
        return;
    }
    uint32_t const quarter = ((c1 - c0 + 3) / 4 + 63) / 64 * 64;
    uint32_t const s0 = min(c0 + wave * quarter, c1);
    uint32_t const s1 = min(s0 + quarter, c1);
    WavePartial w;
    if (s0 < s1) {
        w = decode_wave_d64<kStream>(lds.groups, GroupResolver(P, item.layer, h), item, h, G, c0, s0, s1,
                                     new_token_rows(lds, jv, item.token_count, h, 64));
    } else {
#pragma unroll
        for (uint32_t db = 0; db < 4; ++db) w.acc[db] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
        w.m = -INFINITY;
        w.l = 0.0f;
    }
    // Every wave is done with the group table: its LDS holds the four states,
    // [wave][query column][68 floats: o(64), m, l, pad].
    constexpr uint32_t kRow = 68;
    __syncthreads();
    float* part = reinterpret_cast<float*>(lds.groups);
    {
        uint32_t const l = tid & 63u;
        float* row = part + (wave * 16 + (l & 15u)) * kRow;
#pragma unroll
        for (uint32_t db = 0; db < 4; ++db) {
            *reinterpret_cast<float4_t*>(row + db * 16 + 4 * (l >> 4)) = w.acc[db];
        }
        if (l < 16) {
            row[64] = w.m;
            row[65] = w.l;
        }
    }
    __syncthreads();
    // Thread t merges dims [4 (t % 16), +4) of query column t / 16.
    uint32_t const r = tid >> 4;
    uint32_t const d0 = (tid & 15u) * 4;
    if (r >= G) return;
    float M = -INFINITY;
#pragma unroll
    for (uint32_t v = 0; v < kHeadsPerBlock; ++v) M = fmaxf(M, part[(v * 16 + r) * kRow + 64]);
    float den = 0.0f;
    float4_t o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t v = 0; v < kHeadsPerBlock; ++v) {
        const float* row = part + (v * 16 + r) * kRow;
        float const m = row[64];
        float const c = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M);
        den += c * row[65];
        o += c * *reinterpret_cast<const float4_t*>(row + d0);
    }
    store_partial(item, QH, h * G + r, chunk_index, single, o, d0, M, den, d0 == 0);
}

// Stores the lane's new token for kv heads [h0, h1) of `layer` (a job that
// write_job_valid accepted: one token, one layer, source rows [H][D]), the
// copy-on-write of a replaced partial tail included.  Made by the workgroup
// whose chunk holds the lane's last token, after its own reads: no read of
// the launch takes these positions from the destination page (JobView), so
// nothing waits for the stores.  Every thread of the workgroup calls it.
__device__ void write_token_heads(const PoolView& P, const kimkv_append_job& job, uint32_t layer, uint32_t h0,
                                  uint32_t h1)
{
    uint32_t const D = P.dim;
    uint32_t const dcap = pool_tokens(P, job.dst_kind);
    uint16_t* dst = page_base(P, job.dst_kind, job.dst_slot, dcap);
    uint32_t const tid = threadIdx.x;
    uint32_t const n = job.cow_tokens;
    if (n != 0) {
        uint32_t const scap = pool_tokens(P, job.cow_kind);
        uint16_t const* src = page_base(P, job.cow_kind, job.cow_slot, scap);
        uint32_t const per_head = n * D;
        for (uint32_t i = tid; i < (h1 - h0) * per_head; i += kBlock) {
            uint32_t const h = h0 + i / per_head;
            uint32_t const rem = i % per_head;
            uint32_t const t = rem / D;
            uint32_t const d = rem - t * D;
            uint64_t const sh = head_block(P, scap, layer, h);
            uint64_t const dh = head_block(P, dcap, layer, h);
            dst[dh + k_offset(dcap, D, t, d)] = src[sh + k_offset(scap, D, t, d)];
            dst[dh + v_offset(dcap, D, t, d)] = src[sh + v_offset(scap, D, t, d)];
        }
    }
    for (uint32_t i = tid; i < (h1 - h0) * D; i += kBlock) {
        uint32_t const h = h0 + i / D;
        uint32_t const d = i % D;
        uint64_t const dh = head_block(P, dcap, layer, h);
        dst[dh + k_offset(dcap, D, job.dst_token, d)] = job.src_key[h * D + d];
        dst[dh + v_offset(dcap, D, job.dst_token, d)] = job.src_value[h * D + d];
    }
}

// What a lane's split-K merge needs, written by the decode launch's first
// workgroup of the lane (chunk 0, first head block) so that the merge launch
// reads device memory instead of the launch's items (host memory when the
// engine stages them).  `tag` names the launch: a slot another launch wrote,
// or that no workgroup wrote, does not match and is skipped.
struct DecodeLaneSlot {
    uint16_t* output;
    float* workspace;   // where the lane's partials went
    uint32_t chunks;
    uint32_t lane;
    uint64_t tag;
};
static_assert(sizeof(DecodeLaneSlot) == KIMKV_DECODE_LANE_SLOT_BYTES, "slot size");

// Two waves per SIMD: each wave holds two 64-token steps of K/V operands in
// registers, so a CU keeps as many bytes in flight as four single-buffered
// waves while the compute of one step hides under the loads of the next.
//
// kSplit = false: workgroup = (lane, chunk, four kv heads), wave w takes kv
//   head 4 blockIdx.y + w over the whole chunk.
// kSplit = true: workgroup = (lane, chunk, kv head blockIdx.y); the chunk is
//   cut into four 64-token-aligned quarters, one per wave, and the four
//   online-softmax states are merged through LDS, so a lane that fits one
//   chunk writes its output directly and needs no combine launch.
//
// partials: when non-null, split-K partials of global chunk c go to
// partials + c * QH * (D + 2) instead of the lanes' own workspaces.
// writes: when non-null, lane i's new token (writes[i], token_count 0 for
// none): every chunk reads the positions the job writes from the job's
// sources, and the workgroups of the chunk that holds the lane's last token
// store them after their reads.
// kStream: non-temporal K/V loads (load_kv).
// slots: when non-null, each lane's merge record (DecodeLaneSlot, tagged
// `tag`) for the merge launch.
// kSrc / lanes / sa: where a workgroup gets its lane, item and job (LaneSource
// below); lanes is read only by kRecords launches, items and writes only by
// the others.
// The grid has one workgroup per chunk (x) and head block (y); the merge
// launch follows when gridDim.x > lane_count, and a lane of several chunks
// in a launch without it is reported and skipped.  A lane of no tokens is
// skipped (its output is not written), as the reference's batch kernel does.
// The chunk prefix of a small launch carried in its arguments (kimkv
// launches copy the arguments to device memory with the dispatch), so a
// workgroup finds its lane exactly without reading the prefix from wherever
// the caller staged it; used for launches of up to
// KIMKV_DECODE_ARG_PREFIX_LANES lanes when the caller passes a host copy.
struct ArgPrefix {
    uint32_t v[KIMKV_DECODE_ARG_PREFIX_LANES + 1];
};
struct NoArgPrefix {};

// Where a workgroup finds its lane and reads the lane's item and write job.
enum class LaneSource {
    kGuess,       // items[] and writes[]; lane guessed from the chunk, checked against prefix[]
    kArgPrefix,   // items[] and writes[]; lane from the prefix in the launch arguments
    kRecords,     // item, job and lane built from the chunk's step-constant
                  // kimkv_decode_lane in device memory and the layer arguments
};

// Arguments of a kRecords launch: the prefix and the per-layer addresses.
struct RecordArgs {
    kimkv_decode_layer_args layer;
    TableCache cache;
};


template <LaneSource kSrc>
using SourceArgs = std::conditional_t<kSrc == LaneSource::kGuess, NoArgPrefix,
                                      std::conditional_t<kSrc == LaneSource::kArgPrefix, ArgPrefix, RecordArgs>>;

template <typename T>
__device__ inline T* at_stride(T* base, uint64_t stride, uint32_t i)
{
    return reinterpret_cast<T*>(reinterpret_cast<uintptr_t>(base) + stride * i);
}

// The item and write job of lane i of a kRecords launch: what the engine
// would stage for it, from its step record and the layer's arguments.
__device__ inline void record_lane(const kimkv_decode_lane& r, const kimkv_decode_layer_args& a, uint32_t i,
                                   kimkv_decode_item& item, kimkv_append_job& job)
{
    item.descriptors = r.descriptors;
    item.descriptor_count = r.descriptor_count;
    item.token_count = r.token_count;
    item.layer = a.layer;
    item.query = at_stride(a.query, a.query_stride, i);
    item.workspace = a.workspace != nullptr ? at_stride(a.workspace, a.workspace_stride, i) : nullptr;
    item.output = at_stride(a.output, a.output_stride, i);
    item.attention_scale = a.attention_scale;
    job = kimkv_append_job{};
    if (r.has_write != 0) {
        job.src_key = at_stride(a.key, a.key_stride, i);
        job.src_value = at_stride(a.value, a.value_stride, i);
        job.layer_begin = a.layer;
        job.layer_count = 1;
        job.token_count = 1;
        job.dst_slot = r.dst_slot;
        job.cow_slot = r.cow_slot;
        job.dst_token = r.dst_token;
        job.cow_tokens = r.cow_tokens;
        job.dst_kind = r.dst_kind;
        job.cow_kind = r.cow_kind;
    }
}

template <bool kSplit, bool kStream, LaneSource kSrc>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_kernel(
    PoolView P, const kimkv_decode_item* items, const uint32_t* prefix, uint32_t lane_count, uint32_t chunk_tokens,
    uint32_t QH, float* partials, const kimkv_append_job* writes, DecodeLaneSlot* slots, uint64_t tag,
    const kimkv_decode_lane* lanes, SourceArgs<kSrc> sa)
{
    __shared__ DecodeLds lds;
    __shared__ uint32_t s_lane;
    __shared__ uint32_t s_hit;
    __shared__ TableCacheHeader s_cache_hdr;

    uint32_t const tid = threadIdx.x;
    // One workgroup per chunk with every head (grid.y == 1): each XCD takes a
    // contiguous run of chunks (workgroups are dealt to the XCDs round-robin),
    // so the lanes next to each other in the batch -- forks of one prefix,
    // whose leading chunks read the same pages -- meet in one XCD's L2.
    uint32_t const chunk_id = !kSplit && gridDim.y == 1 ? xcd_logical_index(blockIdx.x, gridDim.x) : blockIdx.x;
    if (lane_count == 0) return;
    uint32_t lane = 0;
    uint32_t lane_first = 0;
    uint32_t lane_end = 0;
    kimkv_decode_item item;
    kimkv_append_job job;
    if constexpr (kSrc == LaneSource::kRecords) {
        // One round trip: the chunk's record and its cached group table (if
        // any), both at addresses that follow from the chunk alone.  (Plain
        // vector values, not arrays or structs, so that they stay in
        // registers: a local aggregate may be placed in LDS by the compiler,
        // which then waits for its load at once to store it there.)
        static_assert(sizeof(kimkv_decode_lane) == 48, "chunk record is 48 bytes");
        static_assert(kTableCachePerThread == 2, "two prefetched entries per thread");
        const uint4* rp = reinterpret_cast<const uint4*>(lanes + chunk_id);
        uint4 const r0 = rp[0];
        uint4 const r1 = rp[1];
        uint4 const r2 = rp[2];
        uint4 hdr = {0u, 0u, 0u, 0u};
        uint2 ent0 = {0u, 0u};
        uint2 ent1 = {0u, 0u};
        if (sa.cache.base != nullptr) {
            const unsigned char* c = sa.cache.base + table_cache_chunk_bytes(sa.cache.stride) * chunk_id;
            const uint2* e = reinterpret_cast<const uint2*>(c + sizeof(TableCacheHeader));
            hdr = *reinterpret_cast<const uint4*>(c);
            if (tid < sa.cache.stride) ent0 = e[tid];
            if (tid + kBlock < sa.cache.stride) ent1 = e[tid + kBlock];
        }
        struct Thirds {
            uint4 a, b, c;
        };
        kimkv_decode_lane const rec = __builtin_bit_cast(kimkv_decode_lane, Thirds{r0, r1, r2});
        lane = rec.lane;
        lane_first = rec.first_chunk;
        lane_end = rec.first_chunk + rec.chunk_count;
        if (!(lane < lane_count && lane_first <= chunk_id && chunk_id < lane_end && lane_end >= lane_first)) {
            report_fault(P, KIMKV_FAULT_DECODE_ITEM);   // the record does not cover this workgroup
            return;
        }
        record_lane(rec, sa.layer, lane, item, job);
        if (sa.cache.base != nullptr) {
            if (tid == 0) s_cache_hdr = __builtin_bit_cast(TableCacheHeader, hdr);
            if (tid < sa.cache.stride) lds.groups[tid] = __builtin_bit_cast(GroupEntry, ent0);
            if (tid + kBlock < sa.cache.stride) lds.groups[tid + kBlock] = __builtin_bit_cast(GroupEntry, ent1);
        }
    } else if constexpr (kSrc == LaneSource::kArgPrefix) {
        // The last lane whose first chunk is <= chunk_id (scalar loads of the
        // launch arguments), then one round trip for its item and job.
        ArgPrefix const& ap = sa;
        uint32_t lo = 0;
        uint32_t hi = lane_count;
        while (hi - lo > 1) {
            uint32_t const mid = (lo + hi) >> 1;
            if (ap.v[mid] <= chunk_id) {
                lo = mid;
            } else {
                hi = mid;
            }
        }
        lane = lo;
        lane_first = ap.v[lane];
        lane_end = ap.v[lane + 1];
        if (!(lane_first <= chunk_id && chunk_id < lane_end)) {   // the prefix does not cover this workgroup
            report_fault(P, KIMKV_FAULT_DECODE_ITEM);
            return;
        }
        item = items[lane];
        job = writes != nullptr ? writes[lane] : kimkv_append_job{};
    } else {
        // The prologue is a chain of dependent global reads, and under full
        // HBM load each costs microseconds while this workgroup streams
        // nothing, so both lookups are guessed and verified in the same round
        // trip.  Lane: guess from the average chunk count per lane (exact
        // when lanes have equal chunk counts), with that lane's item loaded
        // alongside.
        uint32_t const guess = static_cast<uint32_t>(
            min(static_cast<uint64_t>(chunk_id) * lane_count / gridDim.x, static_cast<uint64_t>(lane_count - 1)));
        item = items[guess];
        // The lane's write job comes in the same round trip (kimkv_append_job{}
        // when there is none).
        job = writes != nullptr ? writes[guess] : kimkv_append_job{};
        uint32_t const pg0 = prefix[guess];
        uint32_t const pg1 = prefix[guess + 1];
        if (tid == 0) {
            s_hit = pg0 <= chunk_id && chunk_id < pg1 ? 1u : 0u;
            s_lane = 0xFFFFFFFFu;
        }
        __syncthreads();
        lane = guess;
        if (s_hit == 0) {
            for (uint32_t i = tid; i < lane_count; i += kBlock) {
                if (prefix[i] <= chunk_id && chunk_id < prefix[i + 1]) s_lane = i;
            }
            __syncthreads();
            lane = s_lane;
            if (lane == 0xFFFFFFFFu) {   // the chunk prefix does not cover this workgroup
                report_fault(P, KIMKV_FAULT_DECODE_ITEM);
                return;
            }
            item = items[lane];
            if (writes != nullptr) job = writes[lane];
        }
        lane_first = prefix[lane];
        lane_end = prefix[lane + 1];
    }

    uint32_t const H = P.heads;
    uint32_t const D = P.dim;
    uint32_t const chunk_index = chunk_id - lane_first;
    uint32_t const nchunks = lane_end - lane_first;
    if (partials != nullptr) item.workspace = partials + static_cast<uint64_t>(lane_first) * QH * (D + 2);
    uint32_t const T = item.token_count;
    if (T == 0) return;
    uint32_t const c0 = chunk_index * chunk_tokens;
    // A lane's chunks must lie inside the launch (the merge reads them all).
    if (!decode_item_valid(P, item, QH, nchunks, gridDim.x > lane_count) || c0 >= T || chunk_tokens > kMaxChunk
        || lane_end > gridDim.x) {
        report_fault(P, KIMKV_FAULT_DECODE_ITEM);
        return;
    }
    if (slots != nullptr && chunk_index == 0 && blockIdx.y == 0 && tid == 0) {
        slots[lane] = DecodeLaneSlot{item.output, item.workspace, nchunks, lane, tag};
    }
    uint32_t const c1 = min(c0 + chunk_tokens, T);
    uint32_t const G = QH / H;
    bool const single = nchunks == 1;
    uint32_t const wh0 = kSplit ? blockIdx.y : blockIdx.y * kHeadsPerBlock;
    uint32_t const wh1 = kSplit ? wh0 + 1 : min(H, wh0 + kHeadsPerBlock);
    bool const job_ok = job.token_count != 0 && write_job_valid(P, job, item.layer);
    // The chunk holding the lane's last token stores the job's positions of
    // its kv heads, after its reads.
    bool const writer = job.token_count != 0 && c1 == T && wh0 < H;
    if (writer && !job_ok) report_fault(P, KIMKV_FAULT_APPEND_JOB);
    JobView const jv = job_view(P, job, job_ok);
    if (tid == 0) lds.job = job;   // visible after build_chunk_table's barriers
    bool fast;
    if constexpr (kSrc == LaneSource::kRecords) {
        fast = chunk_table_cached(P, item, QH, c0, c1, lds, jv, sa.cache, chunk_id, s_cache_hdr);
    } else {
        fast = build_chunk_table(P, item, QH, c0, c1, lds, jv);
    }

    uint32_t const wave = tid >> 6;
    if (!kSplit) {
        uint32_t const h = blockIdx.y * kHeadsPerBlock + wave;
        if (h < H && !fast) {
            decode_wave_generic(P, item, h, G, QH, c0, c1, chunk_index, single, &lds.wave_tokens[wave], jv);
        } else if (h < H) {
            WavePartial const w = decode_wave_d64<kStream>(lds.groups, GroupResolver(P, item.layer, h), item, h, G,
                                                           c0, c0, c1, new_token_rows(lds, jv, T, h, 64));
            uint32_t const l = tid & 63u;
            uint32_t const r = l & 15u;
            if (r < G) {
#pragma unroll
                for (uint32_t db = 0; db < 4; ++db) {
                    store_partial(item, QH, h * G + r, chunk_index, single, w.acc[db], db * 16 + 4 * (l >> 4), w.m,
                                  w.l, db == 0 && l < 16);
                }
            }
        }
    } else if (blockIdx.y < H) {
        decode_head_split_chunk<kStream>(P, item, blockIdx.y, QH, c0, c1, chunk_index, single, fast, lds, jv);
    }
    // The job comes back from LDS rather than staying in registers across
    // the streaming loop.
    if (writer && job_ok) write_token_heads(P, lds.job, item.layer, wh0, wh1);
}

// Slices of a lane of T tokens in the guided mode: at most six, and no more
// than T / (D + 2), so the lane's partials (slices * QH * (D + 2) floats)
// never exceed the reference's QH * T float workspace.
__host__ __device__ inline uint32_t guided_slices(uint32_t T, uint32_t D)
{
    uint32_t const cap = T / (D + 2u);
    return cap < 1u ? 1u : (cap < KIMKV_DECODE_GUIDED_SLICES ? cap : KIMKV_DECODE_GUIDED_SLICES);
}

// First token of guided slice k of n: slices of halving length (T/2, T/4,
// ..., the last two equal), starts 64-aligned.
__host__ __device__ inline uint32_t guided_edge(uint32_t T, uint32_t n, uint32_t k)
{
    if (k == 0) return 0;
    if (k >= n) return T;
    return (T - (T >> k)) / 64u * 64u;
}

// Guided persistent decode: gridDim.x workgroups (about two per CU) take
// units from counter[0] until none is left.  Unit u is slice u / pairs of
// (lane, kv head) pair u % pairs, so every pair's longest slice comes first
// and the shortest last: workgroups on CUs that get more bandwidth take more
// units, and the launch ends about one short slice after the work runs out
// instead of when the slowest of a fixed set of workgroups finishes.  Each
// unit is a head-split chunk whose partial goes to the lane's slot k; the
// merge launch combines the slices.  The last workgroup to leave resets the
// counter slot for the next launch that uses it.
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_guided_kernel(
    PoolView P, const kimkv_decode_item* items, const uint32_t* prefix, uint32_t lane_count, uint32_t total_chunks,
    uint32_t QH, float* partials, uint32_t* counter, const kimkv_append_job* writes)
{
    __shared__ DecodeLds lds;
    __shared__ uint32_t s_unit;
    constexpr uint32_t K = KIMKV_DECODE_GUIDED_SLICES;
    uint32_t const tid = threadIdx.x;
    uint32_t const H = P.heads;
    uint32_t const D = P.dim;
    uint32_t const G = QH / H;
    uint32_t const pairs = lane_count * H;
    uint32_t const total = pairs * K;
    for (;;) {
        if (tid == 0) s_unit = atomicAdd(&counter[0], 1u);
        __syncthreads();
        uint32_t const u = s_unit;
        __syncthreads();   // every thread has the unit before thread 0 fetches the next
        if (u >= total) break;
        uint32_t const k = u / pairs;
        uint32_t const pair = u - k * pairs;
        uint32_t const lane = pair / H;
        uint32_t const h = pair - lane * H;
        kimkv_decode_item item = items[lane];
        uint32_t const T = item.token_count;
        if (T == 0) continue;   // skipped, as in decode_kernel
        uint32_t const n = guided_slices(T, D);
        if (k >= n) continue;   // a short lane has fewer slices
        uint32_t const first = prefix[lane];
        if (partials != nullptr) item.workspace = partials + static_cast<uint64_t>(first) * QH * (D + 2);
        uint32_t const c0 = guided_edge(T, n, k);
        uint32_t const c1 = guided_edge(T, n, k + 1);
        if (!decode_item_valid(P, item, QH, n, total_chunks > lane_count) || prefix[lane + 1] - first != n
            || prefix[lane + 1] > total_chunks || c1 - c0 > kMaxChunk) {
            report_fault(P, KIMKV_FAULT_DECODE_ITEM);
            continue;
        }
        kimkv_append_job const job = writes != nullptr ? writes[lane] : kimkv_append_job{};
        bool const job_ok = job.token_count != 0 && write_job_valid(P, job, item.layer);
        bool const writer = job.token_count != 0 && c1 == T;
        if (writer && !job_ok) report_fault(P, KIMKV_FAULT_APPEND_JOB);
        JobView const jv = job_view(P, job, job_ok);
        if (tid == 0) lds.job = job;   // the previous unit ended with a barrier
        if (c0 >= c1) {
            // An empty slice still leaves its partial: weight zero in the merge.
            uint32_t const r = tid >> 4;
            uint32_t const d0 = (tid & 15u) * 4;
            if (r < G) {
                store_partial(item, QH, h * G + r, k, false, float4_t{0.0f, 0.0f, 0.0f, 0.0f}, d0, -INFINITY, 0.0f,
                              d0 == 0);
            }
            continue;
        }
        bool const fast = build_chunk_table(P, item, QH, c0, c1, lds, jv);
        decode_head_split_chunk<true>(P, item, h, QH, c0, c1, k, n == 1, fast, lds, jv);
        // The last slice (never empty) stores the job's positions of head h.
        if (writer && job_ok) write_token_heads(P, lds.job, item.layer, h, h + 1);
        __syncthreads();   // the next unit rebuilds the table in the same LDS
    }
    if (tid == 0) {
        uint32_t const left = atomicAdd(&counter[1], 1u);
        if (left + 1 == gridDim.x) {
            atomicExch(&counter[0], 0u);
            atomicExch(&counter[1], 0u);
        }
    }
}

// Merges the per-chunk partials of every multi-chunk lane.  Block = (lane,
// 4 query heads), one wave per head.  Chunks are taken 64 at a time: lane k
// reads chunk k's (m, l) and every lane reads its kDims dims of the chunks'
// partial rows in the same round of loads, so a lane with up to 64 chunks
// (and D <= 64) is merged after a single memory round trip; rounds of 64
// chunks fold into the running (M, den, acc) like an online softmax.
constexpr unsigned kCombineHeads = 4;

// Where the merge of a record launch finds its lanes: each lane's output
// and partials at base + lane * stride, its chunk count from the chunk
// prefix, all in the launch arguments, so a block's first loads are its
// partials.
struct CombineLaneArgs {
    uint16_t* output;
    uint64_t output_stride;   // bytes
    float* workspace;
    uint64_t workspace_stride;   // bytes
    uint32_t prefix[KIMKV_DECODE_ARG_PREFIX_LANES + 1];
};
struct NoCombineLaneArgs {};

// slots: when non-null, the lanes' merge records the decode launch tagged
// `tag` replace the items and the chunk prefix.  With CombineLaneArgs the
// launch arguments replace all three.
template <uint32_t kDims, typename LaneArgs>
__global__ __launch_bounds__(64 * kCombineHeads) void combine_kernel(PoolView P, const kimkv_decode_item* items,
                                                                    const uint32_t* prefix, uint32_t total_chunks,
                                                                    uint32_t QH, uint32_t D, float* partials,
                                                                    const DecodeLaneSlot* slots, uint64_t tag,
                                                                    LaneArgs la)
{
    constexpr uint32_t kBatch = 64 / kDims;   // partial rows held in registers at once
    uint32_t const lane = blockIdx.x;
    uint32_t const q = blockIdx.y * kCombineHeads + (threadIdx.x >> 6);
    uint32_t const l = threadIdx.x & 63u;
    uint32_t n = 0;
    uint16_t* output = nullptr;
    const float* workspace = nullptr;
    if constexpr (std::is_same_v<LaneArgs, CombineLaneArgs>) {
        // Every argument the block needs is read in one round, before the
        // first test (which names the workspace so the load is not sunk
        // below it).
        n = la.prefix[lane + 1] - la.prefix[lane];
        output = at_stride(la.output, la.output_stride, lane);
        workspace = at_stride(la.workspace, la.workspace_stride, lane);
        if (q >= QH || n <= 1 || workspace == nullptr) return;
    } else if (q >= QH) {
        return;
    } else if (slots != nullptr) {
        DecodeLaneSlot const slot = slots[lane];
        if (slot.tag != tag || slot.lane != lane) return;   // no decode workgroup of this launch wrote it
        n = slot.chunks;
        output = slot.output;
        workspace = slot.workspace;
        if (n <= 1) return;
    } else {
        n = prefix[lane + 1] - prefix[lane];
        if (n <= 1 || prefix[lane + 1] > total_chunks) return;   // decode_kernel reported the latter
        kimkv_decode_item item = items[lane];
        if (partials != nullptr) item.workspace = partials + static_cast<uint64_t>(prefix[lane]) * QH * (D + 2);
        if (!decode_item_valid(P, item, QH, n, true)) return;   // decode_kernel reported it
        output = item.output;
        workspace = item.workspace;
    }
    uint64_t const stride = static_cast<uint64_t>(QH) * (D + 2);
    const float* ws = workspace + static_cast<uint64_t>(q) * (D + 2);
    float M = -INFINITY;
    float den = 0.0f;
    float acc[kDims];
#pragma unroll
    for (uint32_t j = 0; j < kDims; ++j) acc[j] = 0.0f;
    float row[kBatch][kDims];
    auto load_rows = [&](const float* blk, uint32_t b, uint32_t kn) {
#pragma unroll
        for (uint32_t i = 0; i < kBatch; ++i) {
#pragma unroll
            for (uint32_t j = 0; j < kDims; ++j) {
                uint32_t const d = l + 64u * j;
                row[i][j] = b + i < kn && d < D ? blk[static_cast<uint64_t>(b + i) * stride + d] : 0.0f;
            }
        }
    };
    for (uint32_t k0 = 0; k0 < n; k0 += 64) {
        uint32_t const kn = min(64u, n - k0);
        const float* blk = ws + static_cast<uint64_t>(k0) * stride;
        float mk = -INFINITY;
        float lk = 0.0f;
        if (l < kn) {
            mk = blk[static_cast<uint64_t>(l) * stride + D];
            lk = blk[static_cast<uint64_t>(l) * stride + D + 1];
        }
        load_rows(blk, 0, kn);
        float const m_new = fmaxf(M, wave_max(mk));
        float const c = M == -INFINITY ? 0.0f : exp2f(M - m_new);
        M = m_new;
        float const w = l < kn ? exp2f(mk - M) : 0.0f;
        den = den * c + wave_sum(w * lk);
#pragma unroll
        for (uint32_t j = 0; j < kDims; ++j) acc[j] *= c;
        for (uint32_t b = 0; b < kn; b += kBatch) {
            if (b != 0) load_rows(blk, b, kn);
#pragma unroll
            for (uint32_t i = 0; i < kBatch; ++i) {
                float const wk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), static_cast<int>(b + i)));
#pragma unroll
                for (uint32_t j = 0; j < kDims; ++j) acc[j] += wk * row[i][j];
            }
        }
    }
    float const inv = 1.0f / den;
#pragma unroll
    for (uint32_t j = 0; j < kDims; ++j) {
        uint32_t const d = l + 64u * j;
        if (d < D) output[static_cast<uint64_t>(q) * D + d] = __half_as_ushort(__float2half_rn(acc[j] * inv));
    }
}

// Reference MHA attention, fp32 query/output: block = (kv head, layer), one wave.
__global__ __launch_bounds__(64) void reference_attention_kernel(PoolView P, const kimkv_block_desc* desc,
                                                                 uint32_t count, uint32_t T, const float* query,
                                                                 float* output)
{
    __shared__ WaveTokens tokens;
    uint32_t const h = blockIdx.x;
    uint32_t const layer = blockIdx.y;
    uint32_t const lane = threadIdx.x;
    uint32_t const D = P.dim;
    const float* qv = query + (static_cast<uint64_t>(layer) * P.heads + h) * D;
    float const scale = 1.0f / sqrtf(static_cast<float>(D));
    float m_run = -INFINITY;
    float l_run = 0.0f;
    float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t t0 = 0; t0 < T; t0 += 64) {
        uint32_t const t = t0 + lane;
        uint32_t idx = find_descriptor_wave(desc, count, t0);
        const uint16_t* page = nullptr;
        uint32_t cap = 0;
        uint32_t pt = 0;
        if (t < T) {
            while (idx + 1 < count && desc[idx + 1].logical_token_begin <= t) ++idx;
            kimkv_block_desc const e = desc[idx];
            if (t >= e.logical_token_begin && t < e.logical_token_begin + e.valid_tokens
                && e.valid_tokens <= e.page_token_capacity) {
                page = page_base(P, e.kind, e.slot, e.page_token_capacity);
                cap = e.page_token_capacity;
                pt = t - e.logical_token_begin;
            }
        }
        float s = -INFINITY;
        const uint16_t* hb = nullptr;
        if (page != nullptr) {
            hb = page + head_block(P, cap, layer, h);
            float dot = 0.0f;
            for (uint32_t d = 0; d < D; ++d) dot += qv[d] * __half2float(__ushort_as_half(hb[k_offset(cap, D, pt, d)]));
            s = dot * scale;
        }
        float const m_new = fmaxf(m_run, wave_max(s));
        float const alpha = m_new == -INFINITY ? 1.0f : expf(m_run - m_new);
        float const p = (page != nullptr && m_new != -INFINITY) ? expf(s - m_new) : 0.0f;
        l_run = l_run * alpha + wave_sum(p);
        m_run = m_new;
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] *= alpha;
        tokens.p[lane] = p;
        tokens.head[lane] = hb;
        tokens.cap[lane] = cap;
        tokens.pt[lane] = pt;
        __syncthreads();
        uint32_t const nt = min(64u, T - t0);
        for (uint32_t tt = 0; tt < nt; ++tt) {
            float const pp = tokens.p[tt];
            const uint16_t* vb = tokens.head[tt];
            uint32_t const vc = tokens.cap[tt];
            uint32_t const vp = tokens.pt[tt];
            if (vb == nullptr || pp == 0.0f) continue;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint32_t const d = lane + 64u * k;
                if (d < D) o[k] += pp * __half2float(__ushort_as_half(vb[v_offset(vc, D, vp, d)]));
            }
        }
        __syncthreads();
    }
    float const inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t const d = lane + 64u * k;
        if (d < D) output[(static_cast<uint64_t>(layer) * P.heads + h) * D + d] = o[k] * inv;
    }
}

// The work-counter slot of `stream` on this storage: the stream's own slot,
// taken on its first guided launch.  False when every slot already belongs
// to another stream.
bool work_counter_slot(const kimkv_storage* storage, kimkv_stream_t stream, uint32_t* slot)
{
    std::lock_guard<std::mutex> lock(storage->work_counter_mutex);
    for (uint32_t i = 0; i < storage->work_counter_owners; ++i) {
        if (storage->work_counter_stream[i] == stream) {
            *slot = i;
            return true;
        }
    }
    if (storage->work_counter_owners == kWorkCounterSlots) return false;
    *slot = storage->work_counter_owners++;
    storage->work_counter_stream[*slot] = stream;
    return true;
}

// Decode launch (+ split-K merge) shared by both entry points.  `partials`
// replaces the lanes' workspaces when non-null; `timed` lets the benchmark's
// event timing see the launch (its events are created on demand).
kimkv_status launch_decode(const kimkv_storage* storage, const kimkv_decode_item* device_items,
                           const uint32_t* device_chunk_prefix, uint32_t lane_count, uint32_t total_chunks,
                           uint32_t chunk_flags, uint32_t query_heads, kimkv_stream_t stream, float* partials,
                           const kimkv_append_job* writes, bool timed, DecodeLaneSlot* slots = nullptr,
                           const uint32_t* host_prefix = nullptr, const kimkv_decode_lane* lanes = nullptr,
                           const kimkv_decode_layer_args* layer_args = nullptr, TableCache cache = {})
{
    bool const head_split = (chunk_flags & KIMKV_DECODE_HEAD_SPLIT) != 0;
    bool const guided = (chunk_flags & KIMKV_DECODE_GUIDED) != 0;
    uint32_t const chunk_tokens = chunk_flags & ~(KIMKV_DECODE_HEAD_SPLIT | KIMKV_DECODE_GUIDED);
    // Lane records: the merge takes its lanes from the chunk prefix and the
    // layer's addresses in its arguments when the caller gives the prefix,
    // else from the decode launch's lane slots (there are no items to read).
    bool const records = lanes != nullptr;
    if (records && (layer_args == nullptr || lane_count > KIMKV_DECODE_ARG_PREFIX_LANES || guided
                    || (total_chunks > lane_count && slots == nullptr && host_prefix == nullptr)
                    || (total_chunks > lane_count && layer_args->workspace == nullptr))) {
        return KIMKV_INVALID_ARGUMENT;
    }
    if (storage == nullptr || (!records && (device_items == nullptr || device_chunk_prefix == nullptr))
        || lane_count == 0
        || query_heads == 0 || query_heads % storage->layout.kv_heads != 0 || storage->layout.head_dim > 256
        || (head_split && guided)
        || (!guided && (chunk_tokens == 0 || chunk_tokens % 64 != 0 || chunk_tokens > kMaxChunk))) {
        return KIMKV_INVALID_ARGUMENT;
    }
    if (total_chunks == 0) return KIMKV_OK;
    hipStream_t const s = native(stream);
    uint32_t const H = storage->layout.kv_heads;
    uint64_t const units = static_cast<uint64_t>(lane_count) * H * KIMKV_DECODE_GUIDED_SLICES;
    if (guided && (units > 0x7FFFFFFFu || storage->work_counters == nullptr)) return KIMKV_INVALID_ARGUMENT;
    dim3 const grid(total_chunks, head_split ? H : (H + kHeadsPerBlock - 1) / kHeadsPerBlock);
    // The guided kernel writes no merge records.
    if (guided) slots = nullptr;
    // Launch tags are unique in the process, so a slot array shared by
    // several storages still never matches another launch's records.
    static std::atomic<uint64_t> next_tag{1};
    uint64_t const tag = slots != nullptr ? next_tag.fetch_add(1, std::memory_order_relaxed) : 0;
    uint32_t slot = 0;
    if (guided && !work_counter_slot(storage, stream, &slot)) return KIMKV_INVALID_ARGUMENT;
    void* start = nullptr;
    if (timed) kernel_timing_begin(TimedKernel::Decode, s, &start);
    if (guided) {
        uint32_t* counter = storage->work_counters + static_cast<size_t>(slot) * kWorkCounterStride;
        uint64_t const resident = 2ull * (storage->compute_units > 0 ? storage->compute_units : 256);
        auto const workers = static_cast<uint32_t>(units < resident ? units : resident);
        decode_guided_kernel<<<workers, kBlock, 0, s>>>(pool_view(*storage), device_items, device_chunk_prefix,
                                                         lane_count, total_chunks, query_heads, partials, counter,
                                                         writes);
    } else {
        // Streamed K/V loads for long chunks (a workgroup streams at least
        // 2048 tokens) or more than one round of resident workgroups (two
        // per CU); cached loads for the short, latency-bound launches.
        uint64_t const resident = 2ull * (storage->compute_units > 0 ? storage->compute_units : 256);
        bool const stream_loads = chunk_tokens >= 2048 || static_cast<uint64_t>(grid.x) * grid.y > resident;
        PoolView const pv = pool_view(*storage);
        auto go = [&](auto split, auto stream_kv, auto src) {
            constexpr bool kS = decltype(split)::value;
            constexpr bool kT = decltype(stream_kv)::value;
            constexpr LaneSource kL = decltype(src)::value;
            SourceArgs<kL> sa{};
            if constexpr (kL == LaneSource::kArgPrefix) {
                for (uint32_t i = 0; i <= lane_count; ++i) sa.v[i] = host_prefix[i];
            } else if constexpr (kL == LaneSource::kRecords) {
                sa.layer = *layer_args;
                sa.cache = cache;
            }
            decode_kernel<kS, kT, kL><<<grid, kBlock, 0, s>>>(pv, device_items, device_chunk_prefix, lane_count,
                                                              chunk_tokens, query_heads, partials, writes, slots, tag,
                                                              lanes, sa);
        };
        auto pick = [&](auto src) {
            using T_ = std::true_type;
            using F_ = std::false_type;
            if (head_split && stream_loads) go(T_{}, T_{}, src);
            else if (head_split) go(T_{}, F_{}, src);
            else if (stream_loads) go(F_{}, T_{}, src);
            else go(F_{}, F_{}, src);
        };
        if (records) {
            pick(std::integral_constant<LaneSource, LaneSource::kRecords>{});
        } else if (host_prefix != nullptr && lane_count <= KIMKV_DECODE_ARG_PREFIX_LANES) {
            pick(std::integral_constant<LaneSource, LaneSource::kArgPrefix>{});
        } else {
            pick(std::integral_constant<LaneSource, LaneSource::kGuess>{});
        }
    }
    if (timed) kernel_timing_end(TimedKernel::Decode, s, start);
    kimkv_status const status = launch_status();
    if (status != KIMKV_OK) return status;
    if (total_chunks > lane_count) {
        dim3 const cgrid(lane_count, (query_heads + kCombineHeads - 1) / kCombineHeads);
        uint32_t const D = storage->layout.head_dim;
        auto merge = [&](auto la) {
            if (D <= 64) {
                combine_kernel<1><<<cgrid, 64 * kCombineHeads, 0, s>>>(pool_view(*storage), device_items,
                                                                         device_chunk_prefix, total_chunks,
                                                                         query_heads, D, partials, slots, tag, la);
            } else if (D <= 128) {
                combine_kernel<2><<<cgrid, 64 * kCombineHeads, 0, s>>>(pool_view(*storage), device_items,
                                                                         device_chunk_prefix, total_chunks,
                                                                         query_heads, D, partials, slots, tag, la);
            } else {
                combine_kernel<4><<<cgrid, 64 * kCombineHeads, 0, s>>>(pool_view(*storage), device_items,
                                                                         device_chunk_prefix, total_chunks,
                                                                         query_heads, D, partials, slots, tag, la);
            }
        };
        if (records && host_prefix != nullptr) {
            CombineLaneArgs la{};
            la.output = layer_args->output;
            la.output_stride = layer_args->output_stride;
            la.workspace = layer_args->workspace;
            la.workspace_stride = layer_args->workspace_stride;
            for (uint32_t i = 0; i <= lane_count; ++i) la.prefix[i] = host_prefix[i];
            merge(la);
        } else {
            merge(NoCombineLaneArgs{});
        }
        return launch_status();
    }
    return KIMKV_OK;
}

// ---- allocation-free decode: split-K partials in a file-scope array ----------
// One copy per device, held until the process ends.  Host code never passes
// the array's name to a kernel (on the host it is a stand-in, not a device
// address): decode_scratch resolves the device address once per device with
// hipGetSymbolAddress and every launch uses that.
__device__ __align__(256) float scratch[KIMKV_DECODE_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the storage's device, which must be the
// current device (the launch runs there).
kimkv_status decode_scratch(const kimkv_storage* storage, float** out)
{
    *out = nullptr;
    int device = -1;
    kimkv_status const got = record_error(hipGetDevice(&device), KIMKV_RUNTIME_UNAVAILABLE);
    if (got != KIMKV_OK) return got;
    if (device != storage->device || device < 0 || device >= kMaxScratchDevices) return KIMKV_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[device] == nullptr) {
        void* ptr = nullptr;
        kimkv_status const resolved =
            record_error(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), KIMKV_RUNTIME_UNAVAILABLE);
        if (resolved != KIMKV_OK) return resolved;
        if (ptr == nullptr) return KIMKV_RUNTIME_UNAVAILABLE;
        g_scratch_ptr[device] = static_cast<float*>(ptr);
    }
    *out = g_scratch_ptr[device];
    return KIMKV_OK;
}

}  // namespace
}  // namespace kimkv

using namespace kimkv;

extern "C" {

kimkv_status kimkv_decode_plan(const kimkv_storage* storage, const uint32_t* token_counts,
                               uint32_t lane_count, uint32_t query_heads, uint32_t* chunk_tokens,
                               uint32_t* chunk_prefix, uint32_t* total_chunks)
{
    if (storage == nullptr || chunk_tokens == nullptr || chunk_prefix == nullptr || total_chunks == nullptr
        || (lane_count != 0 && token_counts == nullptr) || query_heads == 0) {
        return KIMKV_INVALID_ARGUMENT;
    }
    uint64_t total = 0;
    uint64_t longest = 0;
    for (uint32_t i = 0; i < lane_count; ++i) {
        total += token_counts[i];
        longest = token_counts[i] > longest ? token_counts[i] : longest;
    }
    uint64_t const cus = storage->compute_units > 0 ? static_cast<uint64_t>(storage->compute_units) : 256u;
    uint64_t const H = storage->layout.kv_heads;
    uint64_t const head_blocks = (H + kHeadsPerBlock - 1) / kHeadsPerBlock;
    // Aim for one round of resident workgroups (two per CU): every extra
    // workgroup costs a prologue of dependent reads during which its waves
    // stream nothing, and every extra chunk adds split-K partials to merge.
    // Measured at 256 lanes x 32k tokens (one layer, four kv heads per
    // workgroup): 3 workgroups per CU 1.254 ms, 4: 1.268, 8: 1.315,
    // 16: 1.375; at 128 lanes 2 per CU 0.635 ms, 4: 0.653, 8: 0.686.
    uint64_t const slots = cus * 2;
    uint64_t const per_block = (total * head_blocks + slots - 1) / slots;
    uint64_t const per_head = (total * H + slots - 1) / slots;
    // When four kv heads per workgroup would need split-K but one kv head per
    // workgroup would not, take one head per workgroup with its chunk split
    // over the four waves: same workgroup count, no partials, no merge launch.
    bool const fast_shape = storage->layout.head_dim == 64 && query_heads % H == 0 && query_heads / H <= 16;
    // The guided persistent mode (KIMKV_DECODE_GUIDED) is not chosen here: at
    // 128 lanes x 32k tokens it measured 0.638 ms per launch (six slices) and
    // 0.652 ms (three) against 0.628 ms for one head-split chunk per lane on
    // the same MI355X; callers may still request it explicitly.
    bool head_split = per_block < longest && per_head >= longest && fast_shape;
    // A small batch of lanes up to kWholeLaneMax tokens takes the same form
    // when one workgroup per (lane, kv head) fits one round: each wave then
    // streams at most a quarter of the lane and no merge launch follows (4
    // lanes of 18..1001 tokens: 32.9 - 33.4 us per engine step against 34.0
    // - 35.0 us with the lanes split into 256-token chunks, one kv head per
    // workgroup).
    bool const whole_lanes = !head_split && fast_shape && longest > kMinChunk && longest <= kWholeLaneMax
        && lane_count * H <= slots;
    head_split = head_split || whole_lanes;
    uint64_t target = head_split ? longest : per_block;
    if (target < kMinChunk) target = kMinChunk;
    if (target > kMaxChunk) target = kMaxChunk;
    // Even out the longest lane's chunks, so it has no short last chunk.
    if (longest > target) {
        uint64_t const pieces = (longest + target - 1) / target;
        target = (longest + pieces - 1) / pieces;
    }
    target = (target + 63) / 64 * 64;
    if (target < kMinChunk) target = kMinChunk;
    // Every lane gets at least one chunk (a lane of no tokens is one skipped
    // workgroup), so a launch has more chunks than lanes exactly when some
    // lane is split and needs the merge launch.
    uint64_t acc = 0;
    chunk_prefix[0] = 0;
    for (uint32_t i = 0; i < lane_count; ++i) {
        acc += token_counts[i] == 0 ? 1u : (token_counts[i] + target - 1) / target;
        if (acc > 0x7FFFFFFFu) return KIMKV_INVALID_ARGUMENT;
        chunk_prefix[i + 1] = static_cast<uint32_t>(acc);
    }
    // A batch whose chunks stay within one round of resident workgroups even
    // with one kv head per workgroup takes that form as well: each wave then
    // streams a quarter of the chunk, a shorter chain of dependent loads
    // (4 lanes of 18..1001 tokens in 256-token chunks: 33.3 us per engine
    // step against 36.8 - 37.3 us with four kv heads per workgroup; the
    // 32-lane shared-prefix batch has too many chunks for it).
    if (!head_split && fast_shape && acc * H <= slots) head_split = true;
    *chunk_tokens = static_cast<uint32_t>(target) | (head_split ? KIMKV_DECODE_HEAD_SPLIT : 0u);
    *total_chunks = static_cast<uint32_t>(acc);
    return KIMKV_OK;
}

uint32_t kimkv_decode_lane_chunks(uint32_t token_count, uint32_t chunk_tokens, uint32_t head_dim)
{
    if ((chunk_tokens & KIMKV_DECODE_GUIDED) != 0) return guided_slices(token_count, head_dim);
    chunk_tokens &= ~(KIMKV_DECODE_HEAD_SPLIT | KIMKV_DECODE_GUIDED);
    if (chunk_tokens == 0) return 0;
    if (token_count == 0) return 1;
    return static_cast<uint32_t>((static_cast<uint64_t>(token_count) + chunk_tokens - 1) / chunk_tokens);
}

size_t kimkv_decode_workspace_bytes(uint32_t token_count, uint32_t chunk_tokens, uint32_t query_heads,
                                    uint32_t head_dim)
{
    uint64_t const chunks = kimkv_decode_lane_chunks(token_count, chunk_tokens, head_dim);
    if (chunks <= 1) return 0;
    return static_cast<size_t>(chunks * query_heads * (head_dim + 2ull) * sizeof(float));
}

kimkv_status kimkv_paged_decode_batch(const kimkv_storage* storage, const kimkv_decode_item* device_items,
                                      const uint32_t* device_chunk_prefix, uint32_t lane_count,
                                      uint32_t total_chunks, uint32_t chunk_flags, uint32_t query_heads,
                                      kimkv_stream_t stream)
{
    return kimkv::launch_decode(storage, device_items, device_chunk_prefix, lane_count, total_chunks, chunk_flags,
                                query_heads, stream, nullptr, nullptr, true);
}

kimkv_status kimkv_paged_decode_write_batch(const kimkv_storage* storage, const kimkv_decode_item* device_items,
                                            const uint32_t* device_chunk_prefix, uint32_t lane_count,
                                            uint32_t total_chunks, uint32_t chunk_flags, uint32_t query_heads,
                                            const kimkv_append_job* device_writes, kimkv_stream_t stream)
{
    if (device_writes == nullptr) return KIMKV_INVALID_ARGUMENT;
    return kimkv::launch_decode(storage, device_items, device_chunk_prefix, lane_count, total_chunks, chunk_flags,
                                query_heads, stream, nullptr, device_writes, true);
}

kimkv_status kimkv_paged_decode_write_batch_slots(const kimkv_storage* storage,
                                                  const kimkv_decode_item* device_items,
                                                  const uint32_t* device_chunk_prefix, uint32_t lane_count,
                                                  uint32_t total_chunks, uint32_t chunk_flags, uint32_t query_heads,
                                                  const kimkv_append_job* device_writes, void* device_lane_slots,
                                                  kimkv_stream_t stream)
{
    if (device_writes == nullptr || device_lane_slots == nullptr
        || (reinterpret_cast<uintptr_t>(device_lane_slots) & 15u) != 0) {
        return KIMKV_INVALID_ARGUMENT;
    }
    return kimkv::launch_decode(storage, device_items, device_chunk_prefix, lane_count, total_chunks, chunk_flags,
                                query_heads, stream, nullptr, device_writes, true,
                                static_cast<kimkv::DecodeLaneSlot*>(device_lane_slots));
}

kimkv_status kimkv_paged_decode_write_batch_slots_prefix(const kimkv_storage* storage,
                                                         const kimkv_decode_item* device_items,
                                                         const uint32_t* device_chunk_prefix,
                                                         const uint32_t* host_chunk_prefix, uint32_t lane_count,
                                                         uint32_t total_chunks, uint32_t chunk_flags,
                                                         uint32_t query_heads, const kimkv_append_job* device_writes,
                                                         void* device_lane_slots, kimkv_stream_t stream)
{
    if (device_writes == nullptr || device_lane_slots == nullptr || host_chunk_prefix == nullptr
        || (reinterpret_cast<uintptr_t>(device_lane_slots) & 15u) != 0) {
        return KIMKV_INVALID_ARGUMENT;
    }
    // The copy in the arguments must describe the same launch.
    if (lane_count != 0 && (host_chunk_prefix[0] != 0 || host_chunk_prefix[lane_count] != total_chunks)) {
        return KIMKV_INVALID_ARGUMENT;
    }
    return kimkv::launch_decode(storage, device_items, device_chunk_prefix, lane_count, total_chunks, chunk_flags,
                                query_heads, stream, nullptr, device_writes, true,
                                static_cast<kimkv::DecodeLaneSlot*>(device_lane_slots), host_chunk_prefix);
}

kimkv_status kimkv_paged_decode_lanes(const kimkv_storage* storage, const kimkv_decode_lane* device_chunks,
                                      uint32_t lane_count, uint32_t total_chunks, uint32_t chunk_flags,
                                      uint32_t query_heads, const kimkv_decode_layer_args* args,
                                      const uint32_t* host_chunk_prefix, void* device_lane_slots,
                                      void* device_table_cache, uint64_t table_cache_bytes, uint32_t table_tag,
                                      kimkv_stream_t stream)
{
    if (device_chunks == nullptr || args == nullptr || (reinterpret_cast<uintptr_t>(device_chunks) & 15u) != 0
        || (reinterpret_cast<uintptr_t>(device_lane_slots) & 15u) != 0
        || (reinterpret_cast<uintptr_t>(device_table_cache) & 15u) != 0) {
        return KIMKV_INVALID_ARGUMENT;
    }
    if (host_chunk_prefix != nullptr) {
        // A plan of this launch: starts at 0, ends at total_chunks, every
        // lane at least one chunk.
        if (lane_count > KIMKV_DECODE_ARG_PREFIX_LANES || host_chunk_prefix[0] != 0
            || host_chunk_prefix[lane_count] != total_chunks) {
            return KIMKV_INVALID_ARGUMENT;
        }
        for (uint32_t i = 0; i < lane_count; ++i) {
            if (host_chunk_prefix[i + 1] <= host_chunk_prefix[i]) return KIMKV_INVALID_ARGUMENT;
        }
    }
    kimkv::TableCache cache{};
    if (device_table_cache != nullptr) {
        uint32_t const chunk = chunk_flags & ~(KIMKV_DECODE_HEAD_SPLIT | KIMKV_DECODE_GUIDED);
        uint32_t const stride = (chunk + 7) / 8;
        if (table_tag == 0 || chunk > kimkv::kTableCacheMaxChunk
            || table_cache_bytes / kimkv::table_cache_chunk_bytes(stride) < total_chunks) {
            return KIMKV_INVALID_ARGUMENT;
        }
        // Launch ids: nonzero and unique among the launches a cache sees
        // between two uses of one tag (they wrap after 2^32 launches).
        static std::atomic<uint32_t> next_launch{1};
        uint32_t launch = next_launch.fetch_add(1, std::memory_order_relaxed);
        if (launch == 0) launch = next_launch.fetch_add(1, std::memory_order_relaxed);
        cache = kimkv::TableCache{static_cast<unsigned char*>(device_table_cache), stride, table_tag, launch};
    }
    return kimkv::launch_decode(storage, nullptr, nullptr, lane_count, total_chunks, chunk_flags, query_heads,
                                stream, nullptr, nullptr, true, static_cast<kimkv::DecodeLaneSlot*>(device_lane_slots),
                                host_chunk_prefix, device_chunks, args, cache);
}

uint64_t kimkv_decode_table_cache_bytes(uint32_t total_chunks, uint32_t chunk_flags)
{
    uint32_t const chunk = chunk_flags & ~(KIMKV_DECODE_HEAD_SPLIT | KIMKV_DECODE_GUIDED);
    return static_cast<uint64_t>(total_chunks) * kimkv::table_cache_chunk_bytes((chunk + 7) / 8);
}

kimkv_status kimkv_paged_decode_batch_noalloc(const kimkv_storage* storage, const kimkv_decode_item* device_items,
                                              const uint32_t* device_chunk_prefix, uint32_t lane_count,
                                              uint32_t total_chunks, uint32_t chunk_flags, uint32_t query_heads,
                                              kimkv_stream_t stream)
{
    if (storage == nullptr || query_heads == 0) return KIMKV_INVALID_ARGUMENT;
    // Partials are written only when the launch has more chunks than lanes
    // (the kernel refuses a split lane in any other launch), and then within
    // the first total_chunks partial rows.
    uint64_t const need = static_cast<uint64_t>(total_chunks) * query_heads * (storage->layout.head_dim + 2)
        * sizeof(float);
    if (total_chunks > lane_count && need > KIMKV_DECODE_SCRATCH_BYTES) return KIMKV_INVALID_ARGUMENT;
    float* partials = nullptr;
    kimkv_status const resolved = kimkv::decode_scratch(storage, &partials);
    if (resolved != KIMKV_OK) return resolved;
    return kimkv::launch_decode(storage, device_items, device_chunk_prefix, lane_count, total_chunks, chunk_flags,
                                query_heads, stream, partials, nullptr, false);
}

kimkv_status kimkv_reference_attention(const kimkv_storage* storage, const kimkv_block_desc* device_descriptors,
                                       uint32_t descriptor_count, uint32_t total_tokens, const float* device_query,
                                       float* device_output, kimkv_stream_t stream)
{
    if (storage == nullptr || device_descriptors == nullptr || descriptor_count == 0 || total_tokens == 0
        || device_query == nullptr || device_output == nullptr || storage->layout.head_dim > 256) {
        return KIMKV_INVALID_ARGUMENT;
    }
    dim3 const grid(storage->layout.kv_heads, storage->layout.layers);
    reference_attention_kernel<<<grid, 64, 0, native(stream)>>>(pool_view(*storage), device_descriptors,
                                                                descriptor_count, total_tokens, device_query,
                                                                device_output);
    return launch_status();
}

}  // extern "C"
