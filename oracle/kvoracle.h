/*
 * kvoracle.h -- CPU oracle for the heterogeneous paged-KV data path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference's
 * CPU path and of the data semantics of its device kernels.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only
 * to compute expected results or the CPU baseline: the product path never
 * calls it.
 *
 * Pools here use the REFERENCE page layout [layer][K/V][token][head][dim]
 * (include/kim-kv/core/kv_layout.h:73-90), not the device layout, so the
 * device path is compared through layout-independent results (gathered
 * tensors, attention outputs).
 *
 * Pinning (see tests/test_oracle.py): the fp16 codec against the reference's
 * known-answer vectors (tests/reference/kv_reference_test.cpp:24-43), against
 * numpy float16 over all 65536 codes and random floats, and against the
 * compiled reference (oracle/_ref); attention against closed forms
 * (kv_reference_test.cpp:45-95, tests/cuda/cuda_engine_kv_backend_test.cpp:96-129,
 * :347-492) and against the compiled reference referenceAttention; the page
 * copies against the closed-form generator of tests/cuda/cuda_kv_test.cpp:127-172.
 */
#ifndef KVORACLE_H
#define KVORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kvo_layout {
    uint32_t layers;
    uint32_t kv_heads;
    uint32_t head_dim;
} kvo_layout;

/* Mirrors kimkv_block_desc / DeviceBlockDescriptor (engine_kv.h:100-127). */
typedef struct kvo_desc {
    uint32_t slot;
    uint32_t generation;
    uint32_t logical_token_begin;
    uint16_t valid_tokens;
    uint16_t page_token_capacity;
    uint8_t kind;
    uint8_t reserved[3];
} kvo_desc;

/* Host pools: base + slot * page_elements (src/cuda/kv/storage.cpp:46-68). */
typedef struct kvo_pools {
    kvo_layout layout;
    uint16_t* micro;
    uint16_t* extent;
    uint32_t micro_capacity;
    uint32_t extent_capacity;
    uint16_t micro_tokens;
    uint16_t extent_tokens;
} kvo_pools;

/* fp16 codec: floatToKvScalar / kvScalarToFloat (src/reference/kv_reference.cpp:31-134). */
uint16_t kvo_f32_to_f16(float value);
float kvo_f16_to_f32(uint16_t value);
void kvo_f32_to_f16_array(const float* in, uint16_t* out, size_t n);
void kvo_f16_to_f32_array(const uint16_t* in, float* out, size_t n);

/* Synthetic generator shared with the device (kimkv_synth_value). */
uint64_t kvo_mix64(uint64_t z);
uint16_t kvo_synth(uint64_t seed, uint64_t row, uint32_t col);
uint64_t kvo_kv_row(uint32_t stream, uint32_t layer, uint32_t component, uint32_t token);
void kvo_synth_rows(uint16_t* out, uint64_t count, uint64_t seed, uint64_t row0, uint32_t cols);

/* KvLayout::offset (include/kim-kv/core/kv_layout.h:73-90). */
size_t kvo_offset(const kvo_layout* layout, uint32_t layer, uint32_t component,
                  uint32_t token, uint32_t head, uint32_t dim, uint32_t capacity);
size_t kvo_page_elements(const kvo_layout* layout, uint32_t capacity);

/* Page pointer or NULL (storage.cpp:46-68). */
uint16_t* kvo_page(const kvo_pools* pools, uint32_t kind, uint32_t slot);

/* writeLayerTokenKernel (src/cuda/attention/paged_decode_kernels.cu:65-99):
 * key/value are [H][D]. */
int kvo_write_layer_token(const kvo_pools* pools, uint32_t kind, uint32_t slot,
                          uint32_t page_token, uint32_t layer,
                          const uint16_t* key, const uint16_t* value);

/* copyLayerTokensKernel (paged_decode_kernels.cu:29-63): tokens [0,count) of one layer. */
int kvo_copy_layer_tokens(const kvo_pools* pools, uint32_t src_kind, uint32_t src_slot,
                          uint32_t dst_kind, uint32_t dst_slot, uint32_t count, uint32_t layer);

/* copyPageTokensKernel (src/cuda/kv/page_kernels.cu:46-75): tokens [0,count), all layers. */
int kvo_copy_page_tokens(const kvo_pools* pools, uint32_t src_kind, uint32_t src_slot,
                         uint32_t dst_kind, uint32_t dst_slot, uint32_t count);

/* appendTokensKernel (page_kernels.cu:77-127): input is [L][2][input_tokens][H][D];
 * copies input tokens [src_begin, src_begin+count) to page tokens [dst_begin, ...). */
int kvo_append_tokens(const kvo_pools* pools, const uint16_t* input, uint32_t input_tokens,
                      uint32_t src_begin, uint32_t kind, uint32_t slot,
                      uint32_t dst_begin, uint32_t count);

/* promotionKernel (page_kernels.cu:129-182). */
int kvo_promote(const kvo_pools* pools, const uint32_t micro_slots[8], uint32_t extent_slot);

/* gatherKernel (page_kernels.cu:184-242): out is [L][2][total_tokens][H][D]. */
int kvo_gather(const kvo_pools* pools, const kvo_desc* descs, uint32_t count,
               uint32_t total_tokens, uint16_t* out);

/* pagedAttentionScoresKernel + pagedAttentionOutputKernel
 * (paged_decode_kernels.cu:132-298): GQA decode of one lane and one layer.
 * query/output are [query_heads][D] fp16; kv head = q head / (QH / H);
 * s = (q.k)*scale in fp32, max-subtracted exp, fp16 RNE output. */
int kvo_paged_decode(const kvo_pools* pools, const kvo_desc* descs, uint32_t count,
                     uint32_t token_count, uint32_t layer, uint32_t query_heads,
                     const uint16_t* query, float scale, uint16_t* output);

/* Same as kvo_paged_decode but returns the unrounded fp32 output. */
int kvo_paged_decode_f32(const kvo_pools* pools, const kvo_desc* descs, uint32_t count,
                         uint32_t token_count, uint32_t layer, uint32_t query_heads,
                         const uint16_t* query, float scale, float* output);

/* referenceAttention (kv_reference.cpp:136-234): contiguous MHA with fp32
 * query/output [L][H][D], scale 1/sqrt(D).  Returns 1 on success. */
int kvo_reference_attention(const kvo_layout* layout, const uint16_t* kv, uint32_t token_count,
                            const float* query, float* output);

#ifdef __cplusplus
}
#endif

#endif
