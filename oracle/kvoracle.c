/*
 * kvoracle.c -- CPU oracle (TEST INFRASTRUCTURE ONLY; see kvoracle.h).
 * Each function cites the reference file:line whose behaviour it restates.
 */
#include "kvoracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------
 * fp16 codec -- src/reference/kv_reference.cpp:31-134.
 * IEEE-754 binary16, round-to-nearest-even, subnormals kept, NaN -> 0x7E00
 * with the sign preserved, overflow -> infinity.
 * ------------------------------------------------------------------------- */
static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t kvo_f32_to_f16(float value)
{
    uint32_t const u = f32_bits(value);
    uint16_t const sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t const biased = (u >> 23) & 0xFFu;
    uint32_t frac = u & 0x7FFFFFu;

    if (biased == 0xFFu) {                       /* inf / NaN */
        return (uint16_t)(sign | (frac ? 0x7E00u : 0x7C00u));
    }
    int e = (int)biased - 127 + 15;              /* rebias */
    if (e >= 31) {
        return (uint16_t)(sign | 0x7C00u);
    }
    if (e <= 0) {                                /* subnormal or zero */
        if (e < -10) {
            return sign;
        }
        uint32_t const m = frac | 0x800000u;     /* implicit bit */
        uint32_t const drop = (uint32_t)(14 - e);/* bits shifted out */
        uint32_t q = m >> drop;
        uint32_t const rest = m & ((1u << drop) - 1u);
        uint32_t const half = 1u << (drop - 1u);
        if (rest > half || (rest == half && (q & 1u))) {
            q += 1u;                             /* may carry into the exponent field */
        }
        return (uint16_t)(sign | q);
    }
    uint32_t q = frac >> 13;
    uint32_t const rest = frac & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (q & 1u))) {
        q += 1u;
        if (q == 0x400u) {                       /* mantissa overflow */
            q = 0;
            e += 1;
            if (e >= 31) {
                return (uint16_t)(sign | 0x7C00u);
            }
        }
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | q);
}

float kvo_f16_to_f32(uint16_t value)
{
    uint32_t const sign = ((uint32_t)value & 0x8000u) << 16;
    uint32_t const e = ((uint32_t)value >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)value & 0x3FFu;
    if (e == 0x1Fu) {
        return bits_f32(sign | 0x7F800000u | (m << 13));
    }
    if (e != 0) {
        return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
    }
    if (m == 0) {
        return bits_f32(sign);
    }
    int exp = -14;                               /* normalise a subnormal */
    while ((m & 0x400u) == 0) {
        m <<= 1;
        exp -= 1;
    }
    m &= 0x3FFu;
    return bits_f32(sign | ((uint32_t)(exp + 127) << 23) | (m << 13));
}

void kvo_f32_to_f16_array(const float* in, uint16_t* out, size_t n)
{
    for (size_t i = 0; i < n; ++i) out[i] = kvo_f32_to_f16(in[i]);
}

void kvo_f16_to_f32_array(const uint16_t* in, float* out, size_t n)
{
    for (size_t i = 0; i < n; ++i) out[i] = kvo_f16_to_f32(in[i]);
}

/* ---------------------------------------------------------------------------
 * Synthetic generator (shared definition with kimkv_synth_value).
 * ------------------------------------------------------------------------- */
uint64_t kvo_mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint16_t kvo_synth(uint64_t seed, uint64_t row, uint32_t col)
{
    uint64_t const h = kvo_mix64(kvo_mix64(seed + row * 0x9E3779B97F4A7C15ull) + col);
    int32_t const v = (int32_t)(h & 0xFFFFu) + (int32_t)((h >> 16) & 0xFFFFu)
        + (int32_t)((h >> 32) & 0xFFFFu) + (int32_t)(h >> 48) - 131070;
    return kvo_f32_to_f16((float)v * (1.0f / 32768.0f));
}

uint64_t kvo_kv_row(uint32_t stream, uint32_t layer, uint32_t component, uint32_t token)
{
    return ((uint64_t)(stream & 0xFFFFu) << 48) | ((uint64_t)(layer & 0x7FFFu) << 33)
        | ((uint64_t)(component & 1u) << 32) | (uint64_t)token;
}

void kvo_synth_rows(uint16_t* out, uint64_t count, uint64_t seed, uint64_t row0, uint32_t cols)
{
    for (uint64_t i = 0; i < count; ++i) {
        out[i] = kvo_synth(seed, row0 + i / cols, (uint32_t)(i % cols));
    }
}

/* ---------------------------------------------------------------------------
 * Reference page layout -- include/kim-kv/core/kv_layout.h:31-90.
 * ------------------------------------------------------------------------- */
size_t kvo_offset(const kvo_layout* L, uint32_t layer, uint32_t component,
                  uint32_t token, uint32_t head, uint32_t dim, uint32_t capacity)
{
    return ((((size_t)layer * 2 + component) * capacity + token) * L->kv_heads + head)
        * L->head_dim + dim;
}

size_t kvo_page_elements(const kvo_layout* L, uint32_t capacity)
{
    return (size_t)L->layers * 2 * capacity * L->kv_heads * L->head_dim;
}

static uint32_t page_capacity(const kvo_pools* P, uint32_t kind)
{
    return kind == 0 ? P->micro_tokens : P->extent_tokens;
}

uint16_t* kvo_page(const kvo_pools* P, uint32_t kind, uint32_t slot)
{
    if (kind == 0) {
        if (slot >= P->micro_capacity || P->micro == NULL) return NULL;
        return P->micro + (size_t)slot * kvo_page_elements(&P->layout, P->micro_tokens);
    }
    if (kind == 1) {
        if (slot >= P->extent_capacity || P->extent == NULL) return NULL;
        return P->extent + (size_t)slot * kvo_page_elements(&P->layout, P->extent_tokens);
    }
    return NULL;
}

/* writeLayerTokenKernel -- src/cuda/attention/paged_decode_kernels.cu:65-99. */
int kvo_write_layer_token(const kvo_pools* P, uint32_t kind, uint32_t slot,
                          uint32_t page_token, uint32_t layer,
                          const uint16_t* key, const uint16_t* value)
{
    uint16_t* page = kvo_page(P, kind, slot);
    uint32_t const cap = page_capacity(P, kind);
    const kvo_layout* L = &P->layout;
    if (page == NULL || page_token >= cap || layer >= L->layers) return 0;
    for (uint32_t c = 0; c < 2; ++c) {
        const uint16_t* src = c == 0 ? key : value;
        for (uint32_t h = 0; h < L->kv_heads; ++h) {
            for (uint32_t d = 0; d < L->head_dim; ++d) {
                page[kvo_offset(L, layer, c, page_token, h, d, cap)] = src[h * L->head_dim + d];
            }
        }
    }
    return 1;
}

/* copyLayerTokensKernel -- paged_decode_kernels.cu:29-63. */
int kvo_copy_layer_tokens(const kvo_pools* P, uint32_t src_kind, uint32_t src_slot,
                          uint32_t dst_kind, uint32_t dst_slot, uint32_t count, uint32_t layer)
{
    const uint16_t* src = kvo_page(P, src_kind, src_slot);
    uint16_t* dst = kvo_page(P, dst_kind, dst_slot);
    uint32_t const scap = page_capacity(P, src_kind), dcap = page_capacity(P, dst_kind);
    const kvo_layout* L = &P->layout;
    if (!src || !dst || count > scap || count > dcap || layer >= L->layers) return 0;
    for (uint32_t c = 0; c < 2; ++c)
        for (uint32_t t = 0; t < count; ++t)
            for (uint32_t h = 0; h < L->kv_heads; ++h)
                for (uint32_t d = 0; d < L->head_dim; ++d)
                    dst[kvo_offset(L, layer, c, t, h, d, dcap)] =
                        src[kvo_offset(L, layer, c, t, h, d, scap)];
    return 1;
}

/* copyPageTokensKernel -- src/cuda/kv/page_kernels.cu:46-75. */
int kvo_copy_page_tokens(const kvo_pools* P, uint32_t src_kind, uint32_t src_slot,
                         uint32_t dst_kind, uint32_t dst_slot, uint32_t count)
{
    for (uint32_t l = 0; l < P->layout.layers; ++l) {
        if (!kvo_copy_layer_tokens(P, src_kind, src_slot, dst_kind, dst_slot, count, l)) return 0;
    }
    return 1;
}

/* appendTokensKernel -- page_kernels.cu:77-127. */
int kvo_append_tokens(const kvo_pools* P, const uint16_t* input, uint32_t input_tokens,
                      uint32_t src_begin, uint32_t kind, uint32_t slot,
                      uint32_t dst_begin, uint32_t count)
{
    uint16_t* page = kvo_page(P, kind, slot);
    uint32_t const cap = page_capacity(P, kind);
    const kvo_layout* L = &P->layout;
    if (!page || dst_begin + count > cap || src_begin + count > input_tokens) return 0;
    for (uint32_t l = 0; l < L->layers; ++l)
        for (uint32_t c = 0; c < 2; ++c)
            for (uint32_t t = 0; t < count; ++t)
                for (uint32_t h = 0; h < L->kv_heads; ++h)
                    for (uint32_t d = 0; d < L->head_dim; ++d)
                        page[kvo_offset(L, l, c, dst_begin + t, h, d, cap)] =
                            input[kvo_offset(L, l, c, src_begin + t, h, d, input_tokens)];
    return 1;
}

/* promotionKernel -- page_kernels.cu:129-182: extent token t comes from
 * micro page t / 8, token t % 8. */
int kvo_promote(const kvo_pools* P, const uint32_t micro_slots[8], uint32_t extent_slot)
{
    uint16_t* dst = kvo_page(P, 1, extent_slot);
    const kvo_layout* L = &P->layout;
    uint32_t const mt = P->micro_tokens, et = P->extent_tokens;
    if (!dst || mt * 8 != et) return 0;
    for (uint32_t s = 0; s < 8; ++s) {
        if (!kvo_page(P, 0, micro_slots[s])) return 0;
    }
    for (uint32_t l = 0; l < L->layers; ++l)
        for (uint32_t c = 0; c < 2; ++c)
            for (uint32_t t = 0; t < et; ++t) {
                const uint16_t* src = kvo_page(P, 0, micro_slots[t / mt]);
                for (uint32_t h = 0; h < L->kv_heads; ++h)
                    for (uint32_t d = 0; d < L->head_dim; ++d)
                        dst[kvo_offset(L, l, c, t, h, d, et)] =
                            src[kvo_offset(L, l, c, t % mt, h, d, mt)];
            }
    return 1;
}

/* Descriptor covering a logical token: findDescriptor (paged_decode_kernels.cu:115-130). */
static const kvo_desc* find_desc(const kvo_desc* descs, uint32_t count, uint32_t token)
{
    for (uint32_t i = 0; i < count; ++i) {
        if (token >= descs[i].logical_token_begin
            && token < descs[i].logical_token_begin + descs[i].valid_tokens) {
            return &descs[i];
        }
    }
    return NULL;
}

/* gatherKernel -- page_kernels.cu:184-242. */
int kvo_gather(const kvo_pools* P, const kvo_desc* descs, uint32_t count,
               uint32_t total_tokens, uint16_t* out)
{
    const kvo_layout* L = &P->layout;
    for (uint32_t t = 0; t < total_tokens; ++t) {
        const kvo_desc* e = find_desc(descs, count, t);
        if (e == NULL) return 0;
        const uint16_t* page = kvo_page(P, e->kind, e->slot);
        if (page == NULL) return 0;
        uint32_t const pt = t - e->logical_token_begin;
        for (uint32_t l = 0; l < L->layers; ++l)
            for (uint32_t c = 0; c < 2; ++c)
                for (uint32_t h = 0; h < L->kv_heads; ++h)
                    for (uint32_t d = 0; d < L->head_dim; ++d)
                        out[kvo_offset(L, l, c, t, h, d, total_tokens)] =
                            page[kvo_offset(L, l, c, pt, h, d, e->page_token_capacity)];
    }
    return 1;
}

/* pagedAttentionScoresKernel + pagedAttentionOutputKernel --
 * paged_decode_kernels.cu:132-298 (scale applied after the dot, :197-198). */
int kvo_paged_decode_f32(const kvo_pools* P, const kvo_desc* descs, uint32_t count,
                         uint32_t token_count, uint32_t layer, uint32_t query_heads,
                         const uint16_t* query, float scale, float* output)
{
    const kvo_layout* L = &P->layout;
    uint32_t const H = L->kv_heads, D = L->head_dim;
    if (token_count == 0 || H == 0 || query_heads % H != 0 || layer >= L->layers) return 0;
    uint32_t const group = query_heads / H;
    const uint16_t** kpage = (const uint16_t**)malloc(sizeof(void*) * token_count);
    uint32_t* ptok = (uint32_t*)malloc(sizeof(uint32_t) * token_count);
    uint32_t* pcap = (uint32_t*)malloc(sizeof(uint32_t) * token_count);
    float* scores = (float*)malloc(sizeof(float) * token_count);
    float* qf = (float*)malloc(sizeof(float) * D);
    int ok = kpage && ptok && pcap && scores && qf;
    for (uint32_t t = 0; ok && t < token_count; ++t) {
        const kvo_desc* e = find_desc(descs, count, t);
        kpage[t] = e ? kvo_page(P, e->kind, e->slot) : NULL;
        if (!kpage[t]) { ok = 0; break; }
        ptok[t] = t - e->logical_token_begin;
        pcap[t] = e->page_token_capacity;
    }
    for (uint32_t qh = 0; ok && qh < query_heads; ++qh) {
        uint32_t const kvh = qh / group;
        for (uint32_t d = 0; d < D; ++d) qf[d] = kvo_f16_to_f32(query[(size_t)qh * D + d]);
        float maximum = -INFINITY;
        for (uint32_t t = 0; t < token_count; ++t) {
            float dot = 0.0f;
            for (uint32_t d = 0; d < D; ++d) {
                dot += qf[d] * kvo_f16_to_f32(
                    kpage[t][kvo_offset(L, layer, 0, ptok[t], kvh, d, pcap[t])]);
            }
            scores[t] = dot * scale;
            if (scores[t] > maximum) maximum = scores[t];
        }
        float denominator = 0.0f;
        for (uint32_t t = 0; t < token_count; ++t) {
            scores[t] = expf(scores[t] - maximum);
            denominator += scores[t];
        }
        for (uint32_t d = 0; d < D; ++d) {
            float weighted = 0.0f;
            for (uint32_t t = 0; t < token_count; ++t) {
                weighted += scores[t] * kvo_f16_to_f32(
                    kpage[t][kvo_offset(L, layer, 1, ptok[t], kvh, d, pcap[t])]);
            }
            output[(size_t)qh * D + d] = weighted / denominator;
        }
    }
    free(kpage); free(ptok); free(pcap); free(scores); free(qf);
    return ok;
}

int kvo_paged_decode(const kvo_pools* P, const kvo_desc* descs, uint32_t count,
                     uint32_t token_count, uint32_t layer, uint32_t query_heads,
                     const uint16_t* query, float scale, uint16_t* output)
{
    size_t const n = (size_t)query_heads * P->layout.head_dim;
    float* tmp = (float*)malloc(sizeof(float) * (n ? n : 1));
    if (!tmp) return 0;
    int const ok = kvo_paged_decode_f32(P, descs, count, token_count, layer, query_heads,
                                        query, scale, tmp);
    if (ok) kvo_f32_to_f16_array(tmp, output, n);
    free(tmp);
    return ok;
}

/* referenceAttention -- src/reference/kv_reference.cpp:136-234. */
int kvo_reference_attention(const kvo_layout* L, const uint16_t* kv, uint32_t token_count,
                            const float* query, float* output)
{
    uint32_t const H = L->kv_heads, D = L->head_dim;
    if (token_count == 0 || L->layers == 0 || H == 0 || D == 0) return 0;
    float* scores = (float*)malloc(sizeof(float) * token_count);
    if (!scores) return 0;
    float const scale = 1.0f / sqrtf((float)D);
    int ok = 1;
    for (uint32_t l = 0; ok && l < L->layers; ++l) {
        for (uint32_t h = 0; ok && h < H; ++h) {
            size_t const qb = ((size_t)l * H + h) * D;
            float maximum = -INFINITY;
            for (uint32_t t = 0; t < token_count; ++t) {
                float dot = 0.0f;
                for (uint32_t d = 0; d < D; ++d) {
                    dot += query[qb + d]
                        * kvo_f16_to_f32(kv[kvo_offset(L, l, 0, t, h, d, token_count)]);
                }
                scores[t] = dot * scale;
                if (scores[t] > maximum) maximum = scores[t];
            }
            float denominator = 0.0f;
            for (uint32_t t = 0; t < token_count; ++t) {
                scores[t] = expf(scores[t] - maximum);
                denominator += scores[t];
            }
            if (!(denominator > 0.0f) || !isfinite(denominator)) { ok = 0; break; }
            for (uint32_t d = 0; d < D; ++d) {
                float weighted = 0.0f;
                for (uint32_t t = 0; t < token_count; ++t) {
                    weighted += scores[t]
                        * kvo_f16_to_f32(kv[kvo_offset(L, l, 1, t, h, d, token_count)]);
                }
                output[qb + d] = weighted / denominator;
            }
        }
    }
    free(scores);
    return ok;
}
