// model_kernels.hip -- the dense side of a TinyLlama forward for gfx950:
// embedding gather, RMSNorm, RoPE (fused with the q / k / v split), SwiGLU,
// greedy argmax, seeded weight initialisation, and the linear layers on
// rocBLAS (fp16 in, fp32 accumulate).
//
// Counterparts: src/cuda/model/kernels.cuh:11-119 (launchEmbeddingBatch,
// launchRmsNormBatch, launchRopeBatch, launchResidualAddBatch,
// launchSwiGluBatch, launchArgmaxBatch) and the cuBLAS GEMMs of
// src/cuda/model/runner_support.cpp:207-250.  Rounding points follow the
// reference: every activation is stored as fp16 (round to nearest even), the
// logits stay fp32.  Residual adds are fused into the output GEMM (beta = 1),
// which rounds x + W.a once instead of twice.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hipblaslt/hipblaslt.h>

#include <cmath>
#include <mutex>
#include <tuple>
#include <unordered_map>

#include "device_common.h"
#include "runtime_internal.h"

namespace kimkv {
namespace {

constexpr unsigned kBlock = 256;

__device__ inline float h2f(uint16_t v) { return __half2float(__ushort_as_half(v)); }
__device__ inline uint16_t f2h(float v) { return __half_as_ushort(__float2half_rn(v)); }

__global__ __launch_bounds__(kBlock) void fill_scaled_kernel(uint16_t* out, uint64_t count, uint64_t seed,
                                                             uint64_t row0, uint32_t cols, float scale)
{
    uint64_t const stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < count; i += stride) {
        out[i] = f2h(h2f(synth_f16(seed, row0 + i / cols, static_cast<uint32_t>(i % cols))) * scale);
    }
}

__global__ __launch_bounds__(kBlock) void fill_const_kernel(uint16_t* out, uint64_t count, uint16_t bits)
{
    uint64_t const stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < count; i += stride) out[i] = bits;
}

// One row per workgroup: out[r] = table[ids[r]] (ids checked by the host).
__global__ __launch_bounds__(kBlock) void embed_kernel(const uint16_t* table, const uint32_t* ids, uint32_t hidden,
                                                       uint16_t* out)
{
    uint32_t const r = blockIdx.x;
    const uint16_t* src = table + static_cast<uint64_t>(ids[r]) * hidden;
    uint16_t* dst = out + static_cast<uint64_t>(r) * hidden;
    for (uint32_t i = threadIdx.x; i < hidden; i += kBlock) dst[i] = src[i];
}

__device__ inline float block_sum(float v, float* scratch)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    uint32_t const wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63u) == 0) scratch[wave] = v;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (uint32_t w = 0; w < kBlock / 64; ++w) total += scratch[w];
    __syncthreads();
    return total;
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ inline float lo_f(uint32_t w) { return h2f(static_cast<uint16_t>(w & 0xFFFFu)); }
__device__ inline float hi_f(uint32_t w) { return h2f(static_cast<uint16_t>(w >> 16)); }
__device__ inline uint32_t pack2(float a, float b)
{
    return static_cast<uint32_t>(f2h(a)) | (static_cast<uint32_t>(f2h(b)) << 16);
}

// out[r] = fp16(x[src_r] * rsqrt(mean(x[src_r]^2) + eps) * w), src_r = rows ? rows[r] : r.
// 16-byte vectors when hidden % 8 == 0 (every TinyLlama shape), else scalar.
__global__ __launch_bounds__(kBlock) void rmsnorm_kernel(const uint16_t* x, const uint32_t* rows, const uint16_t* w,
                                                         uint32_t hidden, float eps, uint16_t* out)
{
    __shared__ float scratch[kBlock / 64];
    uint32_t const r = blockIdx.x;
    uint32_t const src = rows != nullptr ? rows[r] : r;
    const uint16_t* in = x + static_cast<uint64_t>(src) * hidden;
    uint16_t* o = out + static_cast<uint64_t>(r) * hidden;
    if ((hidden & 7u) == 0) {
        uint32_t const nv = hidden / 8;
        float sq = 0.0f;
        for (uint32_t i = threadIdx.x; i < nv; i += kBlock) {
            u32x4_t const v = reinterpret_cast<const u32x4_t*>(in)[i];
#pragma unroll
            for (int j = 0; j < 4; ++j) sq += lo_f(v[j]) * lo_f(v[j]) + hi_f(v[j]) * hi_f(v[j]);
        }
        float const scale = 1.0f / sqrtf(block_sum(sq, scratch) / static_cast<float>(hidden) + eps);
        for (uint32_t i = threadIdx.x; i < nv; i += kBlock) {
            u32x4_t const v = reinterpret_cast<const u32x4_t*>(in)[i];
            u32x4_t const g = reinterpret_cast<const u32x4_t*>(w)[i];
            u32x4_t y;
#pragma unroll
            for (int j = 0; j < 4; ++j) y[j] = pack2(lo_f(v[j]) * scale * lo_f(g[j]), hi_f(v[j]) * scale * hi_f(g[j]));
            reinterpret_cast<u32x4_t*>(o)[i] = y;
        }
        return;
    }
    float sq = 0.0f;
    for (uint32_t i = threadIdx.x; i < hidden; i += kBlock) {
        float const v = h2f(in[i]);
        sq += v * v;
    }
    float const scale = 1.0f / sqrtf(block_sum(sq, scratch) / static_cast<float>(hidden) + eps);
    for (uint32_t i = threadIdx.x; i < hidden; i += kBlock) o[i] = f2h(h2f(in[i]) * scale * h2f(w[i]));
}

// qkv row = [q: QH*D | k: KVH*D | v: KVH*D].  Rotates q and k by the row's
// position (pairs (d, d + D/2), angle = pos * theta^(-2d/D)) into q_out / k_out
// and copies v to v_out; each output is [rows][heads * D].  The D/2 angles
// of a row are computed once (LDS) and shared by its QH + KVH heads.
constexpr uint32_t kMaxRopeHalf = 256;

__global__ __launch_bounds__(kBlock) void rope_split_kernel(const uint16_t* qkv, const uint32_t* positions,
                                                            uint32_t QH, uint32_t KVH, uint32_t D, float theta,
                                                            uint16_t* q_out, uint16_t* k_out, uint16_t* v_out)
{
    __shared__ float s_cos[kMaxRopeHalf];
    __shared__ float s_sin[kMaxRopeHalf];
    uint32_t const r = blockIdx.x;
    uint32_t const half = D / 2;
    uint64_t const width = static_cast<uint64_t>(QH + 2 * KVH) * D;
    const uint16_t* row = qkv + r * width;
    float const pos = static_cast<float>(positions[r]);
    for (uint32_t d = threadIdx.x; d < half; d += kBlock) {
        float const angle = pos * powf(theta, -2.0f * static_cast<float>(d) / static_cast<float>(D));
        s_cos[d] = cosf(angle);
        s_sin[d] = sinf(angle);
    }
    __syncthreads();
    uint32_t const pairs = (QH + KVH) * half;
    for (uint32_t p = threadIdx.x; p < pairs; p += kBlock) {
        uint32_t const head = p / half;
        uint32_t const d = p - head * half;
        float const c = s_cos[d];
        float const s = s_sin[d];
        bool const is_q = head < QH;
        uint32_t const h = is_q ? head : head - QH;
        const uint16_t* src = row + (is_q ? 0 : static_cast<uint64_t>(QH) * D) + static_cast<uint64_t>(h) * D;
        uint16_t* dst = (is_q ? q_out + static_cast<uint64_t>(r) * QH * D : k_out + static_cast<uint64_t>(r) * KVH * D)
            + static_cast<uint64_t>(h) * D;
        float const a = h2f(src[d]);
        float const b = h2f(src[d + half]);
        dst[d] = f2h(a * c - b * s);
        dst[d + half] = f2h(b * c + a * s);
    }
    const uint16_t* v = row + static_cast<uint64_t>(QH + KVH) * D;
    uint16_t* vo = v_out + static_cast<uint64_t>(r) * KVH * D;
    if (((KVH * D) & 7u) == 0 && ((QH + KVH) * D & 7u) == 0 && (width & 7u) == 0) {
        for (uint32_t i = threadIdx.x; i < KVH * D / 8; i += kBlock) {
            reinterpret_cast<u32x4_t*>(vo)[i] = reinterpret_cast<const u32x4_t*>(v)[i];
        }
    } else {
        for (uint32_t i = threadIdx.x; i < KVH * D; i += kBlock) vo[i] = v[i];
    }
}

// gu row = [gate: inter | up: inter]; out = fp16(silu(gate) * up); 8 elements per thread.
__global__ __launch_bounds__(kBlock) void swiglu_kernel(const uint16_t* gu, uint32_t inter, uint16_t* out)
{
    uint32_t const r = blockIdx.y;
    const uint16_t* row = gu + static_cast<uint64_t>(r) * 2u * inter;
    uint16_t* o = out + static_cast<uint64_t>(r) * inter;
    if ((inter & 7u) == 0) {
        uint32_t const i = blockIdx.x * kBlock + threadIdx.x;
        if (i >= inter / 8) return;
        u32x4_t const g = reinterpret_cast<const u32x4_t*>(row)[i];
        u32x4_t const u = reinterpret_cast<const u32x4_t*>(row + inter)[i];
        u32x4_t y;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float const g0 = lo_f(g[j]), g1 = hi_f(g[j]);
            y[j] = pack2(g0 / (1.0f + expf(-g0)) * lo_f(u[j]), g1 / (1.0f + expf(-g1)) * hi_f(u[j]));
        }
        reinterpret_cast<u32x4_t*>(o)[i] = y;
        return;
    }
    uint32_t const i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= inter) return;
    float const g = h2f(row[i]);
    o[i] = f2h(g / (1.0f + expf(-g)) * h2f(row[inter + i]));
}

// First index of the row maximum (std::max_element order; NaN never wins).
__global__ __launch_bounds__(kBlock) void argmax_kernel(const float* logits, uint32_t V, uint32_t* out)
{
    __shared__ float sv[kBlock / 64];
    __shared__ uint32_t si[kBlock / 64];
    uint32_t const r = blockIdx.x;
    const float* row = logits + static_cast<uint64_t>(r) * V;
    float best = -INFINITY;
    uint32_t idx = 0xFFFFFFFFu;
    for (uint32_t i = threadIdx.x; i < V; i += kBlock) {
        float const v = row[i];
        if (v > best || (idx == 0xFFFFFFFFu && v == v)) {
            best = v;
            idx = i;
        }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        float const ov = __shfl_xor(best, m);
        uint32_t const oi = __shfl_xor(idx, m);
        if (oi != 0xFFFFFFFFu && (idx == 0xFFFFFFFFu || ov > best || (ov == best && oi < idx))) {
            best = ov;
            idx = oi;
        }
    }
    uint32_t const wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63u) == 0) {
        sv[wave] = best;
        si[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < kBlock / 64; ++w) {
            if (si[w] != 0xFFFFFFFFu && (idx == 0xFFFFFFFFu || sv[w] > best || (sv[w] == best && si[w] < idx))) {
                best = sv[w];
                idx = si[w];
            }
        }
        out[r] = idx == 0xFFFFFFFFu ? 0u : idx;
    }
}

unsigned grid_for(uint64_t count)
{
    uint64_t const b = (count + kBlock - 1) / kBlock;
    return static_cast<unsigned>(b < 65536 ? (b == 0 ? 1 : b) : 65536);
}

// hipBLASLt plans.  y^T (out x rows) = W_cm^T . x_cm in column-major terms,
// W_cm = W^T (in x out, ld = in), x_cm = x^T (in x rows, ld = in).  One
// context per stream (a workspace is only safe for one stream's GEMMs at a
// time); every exact problem (rows, in, out, output type, accumulate) keeps
// one plan: the library's first heuristic choice, or the fastest candidate
// measured by kimkv_linear_tune.
constexpr size_t kLtWorkspace = size_t{64} << 20;

struct LtKey {
    uint32_t rows, in, out;
    uint8_t f32, accumulate;
    bool operator==(LtKey const& o) const
    {
        return std::tie(rows, in, out, f32, accumulate) == std::tie(o.rows, o.in, o.out, o.f32, o.accumulate);
    }
};

struct LtKeyHash {
    size_t operator()(LtKey const& k) const noexcept
    {
        uint64_t h = (uint64_t{k.rows} << 32) ^ (uint64_t{k.in} << 16) ^ k.out ^ (uint64_t{k.f32} << 62)
            ^ (uint64_t{k.accumulate} << 63);
        return static_cast<size_t>(mix64(h));
    }
};

struct LtPlan {
    hipblasLtMatmulDesc_t desc{nullptr};
    hipblasLtMatrixLayout_t a{nullptr}, b{nullptr}, c{nullptr};
    hipblasLtMatmulAlgo_t algo{};
};

struct LtContext {
    void* workspace{nullptr};
    std::unordered_map<LtKey, LtPlan, LtKeyHash> plans;
};

struct LtState {
    std::mutex mutex;
    hipblasLtHandle_t handle{nullptr};
    bool failed{false};
    std::unordered_map<hipStream_t, LtContext> by_stream;
};

LtState& lt_state()
{
    static LtState instance;
    return instance;
}

// Caller holds the state mutex.
LtContext* lt_context(LtState& st, hipStream_t stream)
{
    if (st.handle == nullptr) {
        if (st.failed || hipblasLtCreate(&st.handle) != HIPBLAS_STATUS_SUCCESS) {
            st.failed = true;
            st.handle = nullptr;
            return nullptr;
        }
    }
    auto it = st.by_stream.find(stream);
    if (it != st.by_stream.end()) return &it->second;
    LtContext ctx;
    if (hipMalloc(&ctx.workspace, kLtWorkspace) != hipSuccess) return nullptr;
    return &st.by_stream.emplace(stream, std::move(ctx)).first->second;
}

void lt_destroy(LtPlan& p)
{
    if (p.a != nullptr) hipblasLtMatrixLayoutDestroy(p.a);
    if (p.b != nullptr) hipblasLtMatrixLayoutDestroy(p.b);
    if (p.c != nullptr) hipblasLtMatrixLayoutDestroy(p.c);
    if (p.desc != nullptr) hipblasLtMatmulDescDestroy(p.desc);
    p = LtPlan{};
}

bool lt_describe(LtKey const& k, LtPlan& p)
{
    hipblasOperation_t const ta = HIPBLAS_OP_T;
    hipblasOperation_t const tb = HIPBLAS_OP_N;
    bool ok = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS
        && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) == HIPBLAS_STATUS_SUCCESS
        && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) == HIPBLAS_STATUS_SUCCESS
        && hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16F, k.in, k.out, k.in) == HIPBLAS_STATUS_SUCCESS
        && hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16F, k.in, k.rows, k.in) == HIPBLAS_STATUS_SUCCESS
        && hipblasLtMatrixLayoutCreate(&p.c, k.f32 ? HIP_R_32F : HIP_R_16F, k.out, k.rows, k.out)
            == HIPBLAS_STATUS_SUCCESS;
    if (!ok) lt_destroy(p);
    return ok;
}

// Up to `want` candidate algorithms for the plan's problem, best first.
int lt_candidates(LtState& st, LtPlan const& p, hipblasLtMatmulHeuristicResult_t* out, int want)
{
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return 0;
    size_t ws = kLtWorkspace;
    int got = 0;
    if (hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws))
            != HIPBLAS_STATUS_SUCCESS
        || hipblasLtMatmulAlgoGetHeuristic(st.handle, p.desc, p.a, p.b, p.c, p.c, pref, want, out, &got)
            != HIPBLAS_STATUS_SUCCESS) {
        got = 0;
    }
    hipblasLtMatmulPreferenceDestroy(pref);
    return got;
}

hipblasStatus_t lt_run(LtState& st, LtContext& ctx, LtPlan const& p, hipblasLtMatmulAlgo_t const& algo,
                       const uint16_t* x, const uint16_t* w, void* y, float beta, hipStream_t stream)
{
    float const alpha = 1.0f;
    return hipblasLtMatmul(st.handle, p.desc, &alpha, w, p.a, x, p.b, &beta, y, p.c, y, p.c, &algo, ctx.workspace,
                           kLtWorkspace, stream);
}

bool lt_args_ok(const uint16_t* x, uint32_t in, const uint16_t* w, uint32_t out, void* y, uint32_t rows)
{
    return x != nullptr && w != nullptr && y != nullptr && in != 0 && out != 0 && in <= 0x7FFFFFFFu
        && out <= 0x7FFFFFFFu && rows <= 0x7FFFFFFFu;
}

}  // namespace
}  // namespace kimkv

using namespace kimkv;

extern "C" {

kimkv_status kimkv_fill_rows_scaled(uint16_t* device_out, uint64_t count, uint64_t seed, uint64_t row0, uint32_t cols,
                                    float scale, kimkv_stream_t stream)
{
    if (device_out == nullptr || cols == 0) return KIMKV_INVALID_ARGUMENT;
    if (count == 0) return KIMKV_OK;
    fill_scaled_kernel<<<grid_for(count), kBlock, 0, native(stream)>>>(device_out, count, seed, row0, cols, scale);
    return launch_status();
}

kimkv_status kimkv_fill_f16(uint16_t* device_out, uint64_t count, uint16_t bits, kimkv_stream_t stream)
{
    if (device_out == nullptr) return KIMKV_INVALID_ARGUMENT;
    if (count == 0) return KIMKV_OK;
    fill_const_kernel<<<grid_for(count), kBlock, 0, native(stream)>>>(device_out, count, bits);
    return launch_status();
}

kimkv_status kimkv_model_embed(const uint16_t* table, const uint32_t* device_ids, uint32_t rows, uint32_t hidden,
                               uint16_t* out, kimkv_stream_t stream)
{
    if (table == nullptr || device_ids == nullptr || out == nullptr || hidden == 0) return KIMKV_INVALID_ARGUMENT;
    if (rows == 0) return KIMKV_OK;
    embed_kernel<<<rows, kBlock, 0, native(stream)>>>(table, device_ids, hidden, out);
    return launch_status();
}

kimkv_status kimkv_model_rmsnorm(const uint16_t* x, const uint32_t* device_rows, uint32_t rows, const uint16_t* weight,
                                 uint32_t hidden, float eps, uint16_t* out, kimkv_stream_t stream)
{
    if (x == nullptr || weight == nullptr || out == nullptr || hidden == 0 || !(eps > 0.0f)) {
        return KIMKV_INVALID_ARGUMENT;
    }
    if (rows == 0) return KIMKV_OK;
    rmsnorm_kernel<<<rows, kBlock, 0, native(stream)>>>(x, device_rows, weight, hidden, eps, out);
    return launch_status();
}

kimkv_status kimkv_model_rope_split(const uint16_t* qkv, const uint32_t* device_positions, uint32_t rows,
                                    uint32_t query_heads, uint32_t kv_heads, uint32_t head_dim, float theta,
                                    uint16_t* q_out, uint16_t* k_out, uint16_t* v_out, kimkv_stream_t stream)
{
    if (qkv == nullptr || device_positions == nullptr || q_out == nullptr || k_out == nullptr || v_out == nullptr
        || query_heads == 0 || kv_heads == 0 || head_dim == 0 || head_dim % 2 != 0 || head_dim / 2 > kMaxRopeHalf
        || !(theta > 0.0f)) {
        return KIMKV_INVALID_ARGUMENT;
    }
    if (rows == 0) return KIMKV_OK;
    rope_split_kernel<<<rows, kBlock, 0, native(stream)>>>(qkv, device_positions, query_heads, kv_heads, head_dim,
                                                           theta, q_out, k_out, v_out);
    return launch_status();
}

kimkv_status kimkv_model_swiglu(const uint16_t* gate_up, uint32_t rows, uint32_t intermediate, uint16_t* out,
                                kimkv_stream_t stream)
{
    if (gate_up == nullptr || out == nullptr || intermediate == 0 || rows > 65535) return KIMKV_INVALID_ARGUMENT;
    if (rows == 0) return KIMKV_OK;
    uint32_t const lanes = (intermediate & 7u) == 0 ? intermediate / 8 : intermediate;
    dim3 const grid((lanes + kBlock - 1) / kBlock, rows);
    swiglu_kernel<<<grid, kBlock, 0, native(stream)>>>(gate_up, intermediate, out);
    return launch_status();
}

kimkv_status kimkv_model_argmax(const float* logits, uint32_t rows, uint32_t vocabulary, uint32_t* device_out,
                                kimkv_stream_t stream)
{
    if (logits == nullptr || device_out == nullptr || vocabulary == 0) return KIMKV_INVALID_ARGUMENT;
    if (rows == 0) return KIMKV_OK;
    argmax_kernel<<<rows, kBlock, 0, native(stream)>>>(logits, vocabulary, device_out);
    return launch_status();
}

kimkv_status kimkv_linear(const uint16_t* x, uint32_t rows, uint32_t in_features, const uint16_t* weight,
                          uint32_t out_features, void* y, int y_f32, float beta, kimkv_stream_t stream)
{
    if (!lt_args_ok(x, in_features, weight, out_features, y, rows)) return KIMKV_INVALID_ARGUMENT;
    if (rows == 0) return KIMKV_OK;
    LtState& st = lt_state();
    std::lock_guard<std::mutex> lock(st.mutex);
    LtContext* ctx = lt_context(st, native(stream));
    if (ctx == nullptr) return KIMKV_RUNTIME_UNAVAILABLE;
    LtKey const key{rows, in_features, out_features, static_cast<uint8_t>(y_f32 != 0), static_cast<uint8_t>(beta != 0.0f)};
    auto it = ctx->plans.find(key);
    if (it == ctx->plans.end()) {
        LtPlan p;
        hipblasLtMatmulHeuristicResult_t cand[1];
        if (!lt_describe(key, p)) return KIMKV_RUNTIME_UNAVAILABLE;
        if (lt_candidates(st, p, cand, 1) < 1) {
            lt_destroy(p);
            return KIMKV_SUBMISSION_FAILED;
        }
        p.algo = cand[0].algo;
        it = ctx->plans.emplace(key, p).first;
    }
    hipblasStatus_t const r = lt_run(st, *ctx, it->second, it->second.algo, x, weight, y, beta, native(stream));
    return r == HIPBLAS_STATUS_SUCCESS ? KIMKV_OK : KIMKV_SUBMISSION_FAILED;
}

kimkv_status kimkv_linear_tune(const uint16_t* x, uint32_t rows, uint32_t in_features,
                               const uint16_t* const* weights, uint32_t weight_count, uint32_t out_features, void* y,
                               int y_f32, float beta, kimkv_stream_t stream)
{
    constexpr int kCandidates = 16;
    constexpr int kRounds = 3;   // each candidate's time is its best round: one-off interference does not decide
    constexpr int kReps = 5;
    if (weights == nullptr || weight_count == 0) return KIMKV_INVALID_ARGUMENT;
    for (uint32_t i = 0; i < weight_count; ++i) {
        if (!lt_args_ok(x, in_features, weights[i], out_features, y, rows)) return KIMKV_INVALID_ARGUMENT;
    }
    if (rows == 0) return KIMKV_OK;
    LtState& st = lt_state();
    std::lock_guard<std::mutex> lock(st.mutex);
    hipStream_t const s = native(stream);
    LtContext* ctx = lt_context(st, s);
    if (ctx == nullptr) return KIMKV_RUNTIME_UNAVAILABLE;
    LtKey const key{rows, in_features, out_features, static_cast<uint8_t>(y_f32 != 0), static_cast<uint8_t>(beta != 0.0f)};
    LtPlan p;
    if (!lt_describe(key, p)) return KIMKV_RUNTIME_UNAVAILABLE;
    hipblasLtMatmulHeuristicResult_t cand[kCandidates];
    int const n = lt_candidates(st, p, cand, kCandidates);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (n < 1 || hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
        if (e0 != nullptr) static_cast<void>(hipEventDestroy(e0));
        lt_destroy(p);
        return n < 1 ? KIMKV_SUBMISSION_FAILED : KIMKV_RUNTIME_UNAVAILABLE;
    }
    float time_ms[kCandidates];
    bool usable[kCandidates];
    for (int a = 0; a < n; ++a) {
        time_ms[a] = 0.0f;
        usable[a] = lt_run(st, *ctx, p, cand[a].algo, x, weights[0], y, beta, s) == HIPBLAS_STATUS_SUCCESS;
    }
    for (int round = 0; round < kRounds; ++round) {
        for (int a = 0; a < n; ++a) {
            if (!usable[a]) continue;
            bool ok = hipEventRecord(e0, s) == hipSuccess;
            for (int i = 0; i < kReps && ok; ++i) {
                const uint16_t* w = weights[(static_cast<uint32_t>(round * kReps + i) + static_cast<uint32_t>(a)) % weight_count];
                ok = lt_run(st, *ctx, p, cand[a].algo, x, w, y, beta, s) == HIPBLAS_STATUS_SUCCESS;
            }
            float ms = 0.0f;
            ok = ok && hipEventRecord(e1, s) == hipSuccess && hipEventSynchronize(e1) == hipSuccess
                && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
            if (!ok) {
                usable[a] = false;
            } else if (round == 0 || ms < time_ms[a]) {
                time_ms[a] = ms;
            }
        }
    }
    int best = -1;
    for (int a = 0; a < n; ++a) {
        if (usable[a] && (best < 0 || time_ms[a] < time_ms[best])) best = a;
    }
    static_cast<void>(hipEventDestroy(e0));
    static_cast<void>(hipEventDestroy(e1));
    if (best < 0) {
        lt_destroy(p);
        return KIMKV_SUBMISSION_FAILED;
    }
    p.algo = cand[best].algo;
    auto it = ctx->plans.find(key);
    if (it != ctx->plans.end()) {
        lt_destroy(it->second);
        it->second = p;
    } else {
        ctx->plans.emplace(key, p);
    }
    return KIMKV_OK;
}

}  // extern "C"
