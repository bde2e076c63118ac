/*
 * kimkv_hip.h -- C-ABI of the MI355X (gfx950) paged-KV data path.
 *
 * This is the drop-in seam that replaces the reference's internal launch layer
 * `kimkvcache::cuda_detail::launch*` (src/cuda/kv/kernels.cuh:31-143) and the
 * device-pool part of `CudaKvStorage` (src/cuda/kv/storage.cpp:99-190).
 * Every entry point takes plain pointers, sizes and an opaque stream; no HIP,
 * CUDA or torch types appear in the signatures.  All launches are
 * asynchronous on the given stream (NULL = the device's default stream), like
 * the reference's `CudaStream` (include/kim-kv/cuda/cuda_status.h:13).
 *
 * Device page layout (private to the storage; a page holds as many bytes
 * as the reference's): both pools are one allocation of `layers` regions,
 * region l holding every micro page's layer-l block and then every extent
 * page's, so a launch that works on one layer reads one region.  A page's
 * block of one layer holds, per head, 2*cap*D fp16 values: K for `cap`
 * tokens in 32-dim column blocks, then V transposed ([D][cap], in 32-token
 * column blocks).  The contiguous tensors that cross the API (append input,
 * gather output) keep the reference order [layer][K/V][token][head][dim]
 * (include/kim-kv/core/kv_layout.h:73-90).
 */
#ifndef KIMKV_HIP_H
#define KIMKV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* kimkv_stream_t;

/* Mirrors CudaError (include/kim-kv/cuda/cuda_status.h:29-38). */
typedef enum kimkv_status {
    KIMKV_OK = 0,
    KIMKV_INVALID_ARGUMENT = 1,
    KIMKV_RUNTIME_UNAVAILABLE = 2,
    KIMKV_ALLOCATION_FAILED = 3,
    KIMKV_SUBMISSION_FAILED = 4,
    KIMKV_NOT_READY = 5,
    KIMKV_EXECUTION_FAILED = 6,
    KIMKV_INTERNAL_ERROR = 7
} kimkv_status;

/* Page kinds: PageKind (include/kim-kv/core/page_types.h:8-11). */
#define KIMKV_PAGE_MICRO 0u
#define KIMKV_PAGE_EXTENT 1u

/* Layer/head/dim triple: cuda_detail::DeviceLayout (kernels.cuh:14-18). */
typedef struct kimkv_layout {
    uint32_t layers;
    uint32_t kv_heads;
    uint32_t head_dim;
} kimkv_layout;

/* Page-table entry as the kernels see it.  Same fields, order and size
 * (20 bytes) as the reference DeviceBlockDescriptor
 * (include/kim-kv/engine/engine_kv.h:100-127). */
typedef struct kimkv_block_desc {
    uint32_t slot;
    uint32_t generation;
    uint32_t logical_token_begin;
    uint16_t valid_tokens;
    uint16_t page_token_capacity;
    uint8_t kind;
    uint8_t reserved[3];
} kimkv_block_desc;

/* One lane of a ragged decode launch.  Same fields, order and size (56 bytes)
 * as the reference DevicePagedDecodeBatchItem (engine_kv.h:172-191);
 * `workspace` is the lane's split-K partial scratch (the reference's
 * `device_scores`), sized by kimkv_decode_workspace_bytes(). */
typedef struct kimkv_decode_item {
    const kimkv_block_desc* descriptors;
    uint32_t descriptor_count;
    uint32_t token_count;
    uint32_t layer;
    const uint16_t* query;   /* [query_heads][head_dim] fp16 */
    float* workspace;
    uint16_t* output;        /* [query_heads][head_dim] fp16 */
    float attention_scale;
} kimkv_decode_item;

/* One request's chunk of a multi-token causal prefill: the table holds
 * token_count tokens, of which the last new_tokens are the chunk; new token i
 * attends keys [0, token_count - new_tokens + i].  query / output are
 * [new_tokens][query_heads][head_dim] fp16; query 16-byte and output 8-byte
 * aligned (the kernel's vector accesses).  No reference counterpart (the
 * reference advances a prompt chunk one position at a time). */
typedef struct kimkv_prefill_item {
    const kimkv_block_desc* descriptors;
    uint32_t descriptor_count;
    uint32_t token_count;
    uint32_t new_tokens;
    uint32_t layer;
    const uint16_t* query;
    uint16_t* output;
    float attention_scale;
    uint32_t reserved;
} kimkv_prefill_item;

/* One lane's append.  Writes `token_count` tokens of layers
 * [layer_begin, layer_begin+layer_count) into page (dst_kind, dst_slot) at
 * page token `dst_token`.  Source element (l, t, h, d) of K is read at
 *     src_key + (l-layer_begin)*src_layer_stride + t*src_token_stride + h*D + d
 * and likewise for V.  When cow_tokens != 0, page tokens [0, cow_tokens) of
 * those layers are first copied from page (cow_kind, cow_slot): the
 * partial-tail copy-on-write of src/cuda/engine/transaction.cpp:158-191 and
 * src/cuda/kv/append.cpp:45-96.  Replaces launchCopyLayerTokens,
 * launchWriteLayerToken, launchCopyPageTokens and launchAppendTokens
 * (kernels.cuh:31-55,97-117) with one batched kernel. */
typedef struct kimkv_append_job {
    const uint16_t* src_key;
    const uint16_t* src_value;
    uint64_t src_layer_stride;
    uint32_t src_token_stride;
    uint32_t layer_begin;
    uint32_t layer_count;
    uint32_t token_count;
    uint32_t dst_slot;
    uint32_t cow_slot;
    uint16_t dst_token;
    uint16_t cow_tokens;
    uint8_t dst_kind;
    uint8_t cow_kind;
    uint8_t reserved[2];
} kimkv_append_job;

/* One 8-micro -> 1-extent promotion (PromotionSlots, kernels.cuh:27-29). */
typedef struct kimkv_promotion_job {
    uint32_t micro_slots[8];
    uint32_t extent_slot;
} kimkv_promotion_job;

typedef struct kimkv_storage kimkv_storage;

typedef struct kimkv_storage_info {
    kimkv_layout layout;
    uint32_t micro_capacity;
    uint32_t extent_capacity;
    uint16_t micro_page_tokens;
    uint16_t extent_page_tokens;
    uint64_t micro_page_elements;
    uint64_t extent_page_elements;
    uint64_t micro_reserved_bytes;
    uint64_t extent_reserved_bytes;
    int device;
    int compute_units;
} kimkv_storage_info;

/* ---- runtime / memory --------------------------------------------------- */

/* Number of visible HIP devices (0 when the runtime is unavailable). */
int kimkv_device_count(void);

/* Last native HIP error code seen by this thread (diagnostics only). */
int kimkv_last_native_error(void);

kimkv_status kimkv_device_malloc(void** ptr, size_t bytes);
kimkv_status kimkv_device_free(void* ptr);
kimkv_status kimkv_host_malloc_pinned(void** ptr, size_t bytes);
kimkv_status kimkv_host_free_pinned(void* ptr);
/* Pinned, coherent host memory that kernels read directly (zero-copy):
 * *host_ptr is the host address, *device_ptr the address kernels use.  Free
 * with kimkv_host_free_pinned. */
kimkv_status kimkv_host_malloc_mapped(void** host_ptr, void** device_ptr, size_t bytes);
kimkv_status kimkv_memcpy_h2d_async(void* dst, const void* src, size_t bytes, kimkv_stream_t stream);
kimkv_status kimkv_memcpy_d2h_async(void* dst, const void* src, size_t bytes, kimkv_stream_t stream);
kimkv_status kimkv_memcpy_d2d_async(void* dst, const void* src, size_t bytes, kimkv_stream_t stream);
kimkv_status kimkv_stream_create(kimkv_stream_t* stream);
kimkv_status kimkv_stream_destroy(kimkv_stream_t stream);
kimkv_status kimkv_stream_synchronize(kimkv_stream_t stream);
kimkv_status kimkv_device_synchronize(void);

/* Completion events (the reference's cudaEventRecord/Synchronize at the token
 * boundary, src/cuda/engine/transaction.cpp:84-120). */
/* kind: 0 = a synchronization event, 1 = one that also records timing,
 * KIMKV_EVENT_ORDER_ONLY = a synchronization event whose completion
 * publishes no device memory to the host (no system-scope cache writeback
 * when it is reached): for fences that only tell the host that earlier work
 * has finished reading memory the host wrote. */
#define KIMKV_EVENT_ORDER_ONLY 2
kimkv_status kimkv_event_create(void** event, int kind);
kimkv_status kimkv_event_destroy(void* event);
kimkv_status kimkv_event_record(void* event, kimkv_stream_t stream);
/* Work enqueued on `stream` after this call waits for the event's most
 * recent record (cross-stream ordering without a host wait; the model
 * runner's decode stream joins and leaves its main stream this way). */
kimkv_status kimkv_stream_wait_event(kimkv_stream_t stream, void* event);
kimkv_status kimkv_event_query(void* event);       /* KIMKV_OK or KIMKV_NOT_READY */
kimkv_status kimkv_event_synchronize(void* event);
kimkv_status kimkv_event_elapsed_ms(float* ms, void* start, void* stop);

/* ---- storage ------------------------------------------------------------- */

/* Allocates and zero-fills the micro and extent pools on the current device:
 * CudaKvStorage::CudaKvStorage (src/cuda/kv/storage.cpp:99-190). */
kimkv_status kimkv_storage_create(kimkv_storage** out, kimkv_layout layout,
                                  uint32_t micro_capacity, uint32_t extent_capacity,
                                  uint16_t micro_page_tokens, uint16_t extent_page_tokens);
kimkv_status kimkv_storage_destroy(kimkv_storage* storage);
kimkv_status kimkv_storage_query(const kimkv_storage* storage, kimkv_storage_info* info);
/* Device address of a page: CudaKvStorage::Impl::pagePointer (storage.cpp:46-68).
 * Returns NULL for an out-of-range slot.  The page layout is private to the
 * kernels and layer-major: the address is the page's layer-0 block (K and V^T
 * of every head); its layer-l block lies l layer regions further on (a region
 * holds every page's block of one layer), so a page is not one contiguous
 * range. */
uint16_t* kimkv_storage_page(const kimkv_storage* storage, uint32_t kind, uint32_t slot);

/* Fault bits.  A kernel that finds one of its jobs or items invalid (layer
 * out of range, a page that the storage does not hold, a token range past
 * the page, a null pointer, a multi-chunk decode lane without workspace, a
 * chunk prefix that does not cover the grid) skips it, leaving its output
 * unwritten, and sets the matching bit in the storage's fault word. */
#define KIMKV_FAULT_APPEND_JOB 0x1u
#define KIMKV_FAULT_DECODE_ITEM 0x2u
#define KIMKV_FAULT_PREFILL_ITEM 0x4u
#define KIMKV_FAULT_PROMOTION_JOB 0x8u

/* Waits for `stream`, then reads and clears (one atomic exchange, ordered
 * on `stream` after its earlier work) the storage's fault word into *faults
 * (may be NULL).  Returns KIMKV_INVALID_ARGUMENT when any bit was set, so a
 * direct caller of the launch entry points checks a batch with one call.
 * The word is shared by every stream using the storage: bits set by work on
 * other streams are reported by whichever call reads them first.  No
 * counterpart in the reference (its kernels skip invalid input silently,
 * src/cuda/attention/paged_decode_kernels.cu:101-130). */
kimkv_status kimkv_storage_faults(kimkv_storage* storage, kimkv_stream_t stream, uint32_t* faults);

/* ---- data-path kernels ---------------------------------------------------- */

/* Batched append of `job_count` jobs held in DEVICE memory.  `max_layer_count`
 * is the largest layer_count among the jobs (grid height). */
kimkv_status kimkv_append_batch(const kimkv_storage* storage,
                                const kimkv_append_job* device_jobs, uint32_t job_count,
                                uint32_t max_layer_count, kimkv_stream_t stream);

/* Paged -> contiguous [layer][K/V][token][head][dim] copy of one table
 * (launchGather, kernels.cuh:67-75; gatherKernel page_kernels.cu:184-242).
 * Descriptors are in DEVICE memory, sorted and contiguous from token 0. */
kimkv_status kimkv_gather(const kimkv_storage* storage,
                          const kimkv_block_desc* device_descriptors, uint32_t descriptor_count,
                          uint32_t total_tokens, uint16_t* device_output, kimkv_stream_t stream);

/* Batched micro -> extent promotion of DEVICE jobs
 * (launchPromotion, kernels.cuh:57-65; promotionKernel page_kernels.cu:129-182). */
kimkv_status kimkv_promote_batch(const kimkv_storage* storage,
                                 const kimkv_promotion_job* device_jobs, uint32_t job_count,
                                 kimkv_stream_t stream);

/* One range of a device block table rewritten from a source array:
 * table[first, first + count) = descriptors[source, source + count). */
typedef struct kimkv_descriptor_patch {
    kimkv_block_desc* table;
    uint32_t first;
    uint32_t count;
    uint32_t source;
    uint32_t reserved;
} kimkv_descriptor_patch;

/* Applies `patch_count` patches in one launch.  `patches` and `descriptors`
 * may be device memory or mapped pinned host memory; no two patches may
 * write the same entry.  No counterpart in the reference, which uploads
 * every reserved table whole (HipKvStorage / token_reservation.cpp:74): with
 * per-request tables resident on the device, a token's reservation rewrites
 * only the table's tail entry. */
kimkv_status kimkv_patch_descriptors(const kimkv_descriptor_patch* patches, uint32_t patch_count,
                                     const kimkv_block_desc* descriptors, kimkv_stream_t stream);

/* Set by kimkv_decode_plan in *chunk_tokens when each workgroup should take
 * one KV head and split its chunk over its four waves (merged in the
 * workgroup) instead of taking four KV heads (lanes of one chunk that four
 * heads per workgroup would split, or a batch small enough that its chunks
 * fit one round of resident workgroups either way); the other bits are the
 * chunk length.  Pass the planned value through to kimkv_paged_decode_batch and
 * kimkv_decode_workspace_bytes unchanged. */
#define KIMKV_DECODE_HEAD_SPLIT 0x80000000u

/* Opt-in (kimkv_decode_plan does not choose it) guided persistent mode, set in
 * chunk_tokens by the caller:
 * a lane of T tokens is cut into n = min(KIMKV_DECODE_GUIDED_SLICES,
 * max(1, T / (head_dim + 2))) slices of halving length (T/2, T/4, ...,
 * the last two equal; starts 64-aligned), about two workgroups per CU take
 * (slice, lane, KV head) units from a device counter, longest slices first,
 * and the merge launch combines each lane's slices (a one-slice lane is
 * written directly).  The other bits are ignored in this mode; a lane's
 * chunk count is kimkv_decode_lane_chunks.  The counter belongs to the
 * launch's stream (one of 64 per storage, taken on the stream's first guided
 * launch and kept for the storage's lifetime): guided launches on one stream
 * run in order and never share a counter with another stream's; a guided
 * launch from a 65th stream returns KIMKV_INVALID_ARGUMENT. */
#define KIMKV_DECODE_GUIDED 0x40000000u
#define KIMKV_DECODE_GUIDED_SLICES 6u

/* Chunks (split-K partial slots) of a lane of token_count tokens under a
 * planned chunk_tokens value (flags included): the chunk prefix of a launch
 * is the running sum of this over its lanes.  A lane of no tokens has one
 * chunk (a workgroup that skips it), so a launch has more chunks than lanes
 * exactly when some lane is split; the decode launches the split-K merge on
 * that condition and reports (KIMKV_FAULT_DECODE_ITEM) a split lane in a
 * launch with no more chunks than lanes. */
uint32_t kimkv_decode_lane_chunks(uint32_t token_count, uint32_t chunk_tokens, uint32_t head_dim);

/* Split-K planning for a ragged decode batch.  Given the lanes' token counts
 * (host array), picks the chunk length (a multiple of 64 tokens, 256..65536,
 * possibly with KIMKV_DECODE_HEAD_SPLIT set) and fills
 * chunk_prefix[0..lane_count] (host array) with the running chunk count
 * (kimkv_decode_lane_chunks per lane).  Returns the total chunk count in
 * *total_chunks.  A lane of no tokens is skipped by the decode (its output
 * is not written), as the reference's batch kernel skips it. */
kimkv_status kimkv_decode_plan(const kimkv_storage* storage, const uint32_t* token_counts,
                               uint32_t lane_count, uint32_t query_heads,
                               uint32_t* chunk_tokens, uint32_t* chunk_prefix,
                               uint32_t* total_chunks);

/* Workspace bytes one lane needs for a given token count and chunk length
 * (0 when the lane fits one chunk).  Never larger than the reference's
 * score workspace requirement query_heads*token_count*4
 * (src/cuda/engine/transaction.cpp:56-64). */
size_t kimkv_decode_workspace_bytes(uint32_t token_count, uint32_t chunk_tokens,
                                    uint32_t query_heads, uint32_t head_dim);

/* Fused split-K GQA paged decode attention over a ragged batch: replaces
 * launchPagedDecodeAttention / launchPagedDecodeAttentionBatch
 * (kernels.cuh:119-143; paged_decode_kernels.cu:132-474,533-617).
 * q head j reads kv head j / (query_heads / kv_heads); s = (q.k) * scale with
 * fp32 accumulation; softmax; fp16 round-to-nearest-even output.
 * `device_items` and `device_chunk_prefix` live in memory the device reads
 * (device memory, or mapped host memory as the engine stages them). */
kimkv_status kimkv_paged_decode_batch(const kimkv_storage* storage,
                                      const kimkv_decode_item* device_items,
                                      const uint32_t* device_chunk_prefix,
                                      uint32_t lane_count, uint32_t total_chunks,
                                      uint32_t chunk_tokens, uint32_t query_heads,
                                      kimkv_stream_t stream);

/* kimkv_paged_decode_batch with each lane's new token written in the same
 * launch: device_writes[i] (memory the device reads) is lane i's
 * single-token append job for this layer (token_count 1, layer_count 1,
 * layer_begin = the item's layer, source rows [kv_heads][head_dim], its
 * destination normally the lane's last table entry, optionally a
 * copy-on-write source of cow_tokens <= dst_token tokens), or token_count 0
 * for none.  Equals kimkv_append_batch of the jobs followed by
 * kimkv_paged_decode_batch, in one launch: every read of a position the job
 * writes takes it from the job's source (copied positions from the
 * copy-on-write page, dst_token from the source rows), and the workgroups
 * whose chunk holds the lane's last token store the job's positions for
 * their KV heads after their reads, so no read waits for a store and a
 * copied tail may span chunks (any page size).  Outputs are bit-identical to
 * the two-launch form, except for a job copying fewer than dst_token tokens
 * (then within the decode tolerance).  A page a job writes may be read, in
 * the same launch, only by that job's own lane.  No counterpart in the
 * reference, which launches writeLayer and attendLayer separately
 * (src/cuda/engine/transaction.cpp); the engine's batched token path uses it
 * for writeLayerBatch + attendLayerBatch of a layer.  A job that names no
 * page of the storage sets KIMKV_FAULT_APPEND_JOB and is skipped. */
kimkv_status kimkv_paged_decode_write_batch(const kimkv_storage* storage,
                                            const kimkv_decode_item* device_items,
                                            const uint32_t* device_chunk_prefix, uint32_t lane_count,
                                            uint32_t total_chunks, uint32_t chunk_flags,
                                            uint32_t query_heads, const kimkv_append_job* device_writes,
                                            kimkv_stream_t stream);

/* Bytes per lane of kimkv_paged_decode_write_batch_slots's merge records. */
#define KIMKV_DECODE_LANE_SLOT_BYTES 32u

/* kimkv_paged_decode_write_batch whose split-K merge reads no launch item:
 * device_lane_slots (lane_count x KIMKV_DECODE_LANE_SLOT_BYTES bytes of
 * device memory, 16-byte aligned, contents ignored) receives from the decode
 * launch what each lane's merge needs (output, partials, chunk count, tagged
 * with the launch), and the merge launch reads that instead of the items and
 * the chunk prefix.  For callers whose items live in host memory the device
 * reads directly (the engine's staged batches): the merge then starts
 * without a round trip to the host.  Same results as
 * kimkv_paged_decode_write_batch.  No counterpart in the reference. */
kimkv_status kimkv_paged_decode_write_batch_slots(const kimkv_storage* storage,
                                                  const kimkv_decode_item* device_items,
                                                  const uint32_t* device_chunk_prefix, uint32_t lane_count,
                                                  uint32_t total_chunks, uint32_t chunk_flags,
                                                  uint32_t query_heads, const kimkv_append_job* device_writes,
                                                  void* device_lane_slots, kimkv_stream_t stream);

/* Largest lane count whose chunk prefix kimkv_paged_decode_write_batch_slots_prefix
 * carries in the launch's arguments. */
#define KIMKV_DECODE_ARG_PREFIX_LANES 64u

/* kimkv_paged_decode_write_batch_slots with host_chunk_prefix, the same
 * chunk prefix (lane_count + 1 entries) in host memory: for launches of up
 * to KIMKV_DECODE_ARG_PREFIX_LANES lanes the library copies it into the
 * launch's arguments, and each workgroup finds its lane from them with no
 * read of device_chunk_prefix, so when the caller stages the launch data in
 * mapped host memory (the engine) a workgroup's lane lookup costs no round
 * trip to the host and no scan of the prefix; larger launches behave as
 * kimkv_paged_decode_write_batch_slots.  host_chunk_prefix must start at 0
 * and end at total_chunks (else KIMKV_INVALID_ARGUMENT, nothing launched) and
 * equal device_chunk_prefix.  Same results.  No counterpart in the
 * reference. */
kimkv_status kimkv_paged_decode_write_batch_slots_prefix(const kimkv_storage* storage,
                                                         const kimkv_decode_item* device_items,
                                                         const uint32_t* device_chunk_prefix,
                                                         const uint32_t* host_chunk_prefix, uint32_t lane_count,
                                                         uint32_t total_chunks, uint32_t chunk_flags,
                                                         uint32_t query_heads, const kimkv_append_job* device_writes,
                                                         void* device_lane_slots, kimkv_stream_t stream);

/* One chunk of a batched decode launch, with what stays the same for every
 * layer of a token step: its lane's block table and token count, the
 * destination of the lane's single-token write (the write job of
 * kimkv_paged_decode_write_batch without its per-layer source rows), and
 * where the chunk sits (its lane, the lane's first chunk in the launch and
 * the lane's chunk count: the planned chunk prefix, per chunk).  48 bytes;
 * kept by the caller in device memory across the step's layers. */
typedef struct kimkv_decode_lane {
    const kimkv_block_desc* descriptors;
    uint32_t descriptor_count;
    uint32_t token_count;
    uint32_t dst_slot;       /* the write, when has_write != 0 */
    uint32_t cow_slot;
    uint16_t dst_token;
    uint16_t cow_tokens;
    uint8_t dst_kind;
    uint8_t cow_kind;
    uint8_t has_write;
    uint8_t reserved;
    uint32_t lane;
    uint32_t first_chunk;
    uint32_t chunk_count;
    uint32_t reserved2;
} kimkv_decode_lane;

/* The per-layer part of such a launch: lane i reads its query at
 * query + i * query_stride, writes output + i * output_stride, uses workspace
 * + i * workspace_stride when it has more than one chunk, and its write job
 * takes its new K and V rows ([kv_heads][head_dim] fp16) from key + i *
 * key_stride and value + i * value_stride (strides in bytes; arithmetic
 * modulo 2^64, so a negative stride works). */
typedef struct kimkv_decode_layer_args {
    uint32_t layer;
    float attention_scale;
    const uint16_t* query;
    uint64_t query_stride;
    uint16_t* output;
    uint64_t output_stride;
    float* workspace;
    uint64_t workspace_stride;
    const uint16_t* key;
    uint64_t key_stride;
    const uint16_t* value;
    uint64_t value_stride;
} kimkv_decode_layer_args;

/* kimkv_paged_decode_write_batch_slots with each chunk's item and write job
 * assembled in the kernel from device_chunks[chunk] (device memory, 16-byte
 * aligned, one kimkv_decode_lane per chunk of the launch: total_chunks
 * records, the chunks of a lane consecutive) and *args (copied into the
 * launch's arguments): a workgroup's only read before its block table is its
 * chunk's record, whose address follows from the workgroup alone, where the
 * item form finds its lane in the chunk prefix and reads the caller's items
 * and jobs (in mapped host memory when the engine stages them, a round trip
 * to the host).  For a caller whose lanes' queries, outputs, workspaces and
 * new rows are evenly spaced (base + lane * stride), which keeps the records
 * across a step's layers.  lane_count at most KIMKV_DECODE_ARG_PREFIX_LANES;
 * not with KIMKV_DECODE_GUIDED.  When total_chunks > lane_count the split-K
 * merge needs each lane's chunk count: from host_chunk_prefix (optional,
 * NULL for none; lane_count + 1 entries in host memory, 0 first,
 * total_chunks last, strictly increasing, the plan the records were made
 * from), which travels in the merge launch's arguments with the layer's
 * output and workspace bases, so its first reads are the partials; else
 * from device_lane_slots, which is then required.  A record that names a lane past lane_count or a chunk
 * range that does not hold its own chunk, or lies outside the launch, is
 * reported (KIMKV_FAULT_DECODE_ITEM) and skipped.
 * device_table_cache (optional, NULL for none; 16-byte aligned, at least
 * kimkv_decode_table_cache_bytes(total_chunks, chunk_flags) bytes of device
 * memory; chunks of at most 4096 tokens): a cache of each chunk's group
 * table, the page lookups a workgroup derives from its lane's descriptors.
 * They are the same for every layer of a token step, so the step's first
 * launch with a given nonzero table_tag stores them and later launches with
 * that tag read them in the same round trip as the chunk record instead of
 * reading the descriptors.  A tag must not have been stored in this cache by
 * a launch whose records, block-table contents or chunk_flags differ (a
 * fresh tag per token step, and a cache zeroed before first use, keep that),
 * and launches sharing a cache must not overlap (one stream).
 * Anything else returns KIMKV_INVALID_ARGUMENT and launches nothing.  Same
 * results as the item form with the same items, jobs and plan.  No
 * counterpart in the reference. */
kimkv_status kimkv_paged_decode_lanes(const kimkv_storage* storage, const kimkv_decode_lane* device_chunks,
                                      uint32_t lane_count, uint32_t total_chunks, uint32_t chunk_flags,
                                      uint32_t query_heads, const kimkv_decode_layer_args* args,
                                      const uint32_t* host_chunk_prefix, void* device_lane_slots,
                                      void* device_table_cache, uint64_t table_cache_bytes, uint32_t table_tag,
                                      kimkv_stream_t stream);
/* Bytes of the table cache of kimkv_paged_decode_lanes for a launch of
 * total_chunks chunks planned with chunk_flags.  No counterpart in the
 * reference. */
uint64_t kimkv_decode_table_cache_bytes(uint32_t total_chunks, uint32_t chunk_flags);

/* Size of the device scratch array of kimkv_paged_decode_batch_noalloc. */
#define KIMKV_DECODE_SCRATCH_BYTES (16u << 20)

/* kimkv_paged_decode_batch for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, kernels and
 * results; the items' `workspace` pointers are ignored: split-K partials go
 * to a file-scope device array of KIMKV_DECODE_SCRATCH_BYTES bytes (one per
 * device, held until the process ends), which a batch needs only when it
 * has more chunks than lanes (some lane is split; see
 * kimkv_decode_lane_chunks), then total_chunks * query_heads * (head_dim + 2)
 * * 4 bytes of it (16 MiB = 1985 chunks at 32 query heads x 64 dims).
 * KIMKV_INVALID_ARGUMENT for a larger batch or when the storage's device is
 * not the current device; nothing is launched then.  Calls no allocating
 * routine.  Every call on a device shares its array, so calls that overlap
 * on one device (different streams, or threads) race: serialize them.  The
 * array keeps the last call's partials; nothing in it needs clearing (every
 * chunk writes its whole partial before the merge reads it). */
kimkv_status kimkv_paged_decode_batch_noalloc(const kimkv_storage* storage,
                                              const kimkv_decode_item* device_items,
                                              const uint32_t* device_chunk_prefix,
                                              uint32_t lane_count, uint32_t total_chunks,
                                              uint32_t chunk_tokens, uint32_t query_heads,
                                              kimkv_stream_t stream);

/* New tokens handled by one prefill workgroup (per KV head) for this
 * storage's shape and query head count: items need
 * ceil(new_tokens / this) workgroups each.  0 for an invalid head count. */
uint32_t kimkv_prefill_tokens_per_block(const kimkv_storage* storage, uint32_t query_heads);

/* Multi-token causal GQA paged attention (chunked prefill) for a batch of
 * items: block_prefix[0..item_count] is the running workgroup count
 * (kimkv_prefill_tokens_per_block), total_blocks its last entry.  Same
 * arithmetic as kimkv_paged_decode_batch applied to each new token: the
 * output of new token i equals a decode of the first
 * token_count - new_tokens + i + 1 tokens with that token's query. */
kimkv_status kimkv_paged_prefill_batch(const kimkv_storage* storage, const kimkv_prefill_item* device_items,
                                       const uint32_t* device_block_prefix, uint32_t item_count,
                                       uint32_t total_blocks, uint32_t query_heads, kimkv_stream_t stream);

/* One workgroup of an ordered prefill launch: new tokens
 * [block * tokens_per_block, (block + 1) * tokens_per_block) of item `item`
 * for KV head `head`; item == 0xFFFFFFFF marks an idle slot. */
typedef struct kimkv_prefill_block {
    uint32_t item;
    uint16_t head;
    uint16_t block;
} kimkv_prefill_block;

/* Host-side placement of a prefill batch (pure host code): fills
 * order[0 .. *order_count) with every (item, KV head, block) of the batch,
 * laid out for kimkv_paged_prefill_ordered so that each XCD (workgroup w of
 * the launch runs on XCD w % 8) receives a share of (item, head) pairs of
 * about equal total work (their K/V then stays in one L2), and inside an XCD
 * the heaviest blocks share compute units with the lightest.  token_counts[i]
 * and new_tokens[i] are item i's; compute_units is the device's (the
 * storage's kimkv_storage_info).  KIMKV_INVALID_ARGUMENT when capacity is too
 * small (*order_count then holds the size needed).  No counterpart in the
 * reference. */
kimkv_status kimkv_prefill_order(uint32_t kv_heads, uint32_t head_dim, uint32_t query_heads, uint32_t compute_units,
                                 const uint32_t* token_counts, const uint32_t* new_tokens, uint32_t item_count,
                                 kimkv_prefill_block* order, uint32_t capacity, uint32_t* order_count);

/* kimkv_paged_prefill_batch with the workgroup placement of
 * kimkv_prefill_order (device_order in memory the device reads, order_count
 * entries; results are identical to the unordered launch). */
kimkv_status kimkv_paged_prefill_ordered(const kimkv_storage* storage, const kimkv_prefill_item* device_items,
                                         uint32_t item_count, const kimkv_prefill_block* device_order,
                                         uint32_t order_count, uint32_t query_heads, kimkv_stream_t stream);

/* Reference attention over one table (the comparator of the reference's
 * launchAttentionScores / launchAttentionOutput, kernels.cuh:77-95, and of the
 * CPU referenceAttention, src/reference/kv_reference.cpp:136-234): MHA with
 * query head h on kv head h, fp32 query/output [layers][kv_heads][head_dim],
 * scale 1/sqrt(head_dim), fp32 accumulation, all layers. */
kimkv_status kimkv_reference_attention(const kimkv_storage* storage,
                                       const kimkv_block_desc* device_descriptors, uint32_t descriptor_count,
                                       uint32_t total_tokens, const float* device_query, float* device_output,
                                       kimkv_stream_t stream);

/* Summed duration (ms) and count of the decode kernels timed since the last
 * call, measured with events on the launch stream; for the benchmark's
 * roofline.  `enable` > 0 times every enable-th launch from now on (the events
 * around a launch cost the stream a few microseconds), 0 stops timing. */
kimkv_status kimkv_decode_timing(int enable, double* total_ms, uint64_t* launches);
/* The same for the chunked-prefill attention kernel (same `enable`). */
kimkv_status kimkv_prefill_timing(int enable, double* total_ms, uint64_t* launches);
/* The same for the page-append kernel (kimkv_append_batch launches). */
kimkv_status kimkv_append_timing(int enable, double* total_ms, uint64_t* launches);
/* Time (ms) during which at least one timed decode launch was running, over
 * the window the last kimkv_decode_timing call closed: the union of the
 * launches' intervals.  Launches on several streams overlap, so this is less
 * than their summed duration; with every launch timed it is the time the
 * decode kernel occupied the GPU.  No counterpart in the reference (benchmark
 * instrumentation). */
kimkv_status kimkv_decode_timing_busy(double* busy_ms);

/* ---- dense TinyLlama layers (the model runner's device side) --------------
 * Counterparts of src/cuda/model/kernels.cuh:11-119 and the cuBLAS calls of
 * src/cuda/model/runner_support.cpp:207-250.  Activations are fp16 rows,
 * stored with round-to-nearest-even; all accumulation is fp32. */

/* y[rows][out] = x[rows][in] . weight[out][in]^T + beta * y (hipBLASLt, fp32
 * accumulate).  y is fp16 (y_f32 = 0) or fp32 (y_f32 != 0); beta = 1 with
 * y = the residual stream fuses the residual add.  Each exact problem (rows,
 * in, out, output type, beta != 0) keeps one algorithm per stream: the
 * library's first heuristic choice unless kimkv_linear_tune chose one. */
kimkv_status kimkv_linear(const uint16_t* x, uint32_t rows, uint32_t in_features, const uint16_t* weight,
                          uint32_t out_features, void* y, int y_f32, float beta, kimkv_stream_t stream);
/* Times the library's leading candidates for this exact problem (the stream
 * is synchronized; y is overwritten or accumulated into several times, so
 * pass scratch contents) and makes the fastest the one kimkv_linear uses for
 * the problem on this stream.  Successive timed products cycle through the
 * weight_count weight matrices (e.g. every layer's), so the weights are read
 * from HBM as in a forward pass, not from a warm cache.  No counterpart in
 * the reference (cuBLAS picks its own algorithm). */
kimkv_status kimkv_linear_tune(const uint16_t* x, uint32_t rows, uint32_t in_features,
                               const uint16_t* const* weights, uint32_t weight_count, uint32_t out_features, void* y,
                               int y_f32, float beta, kimkv_stream_t stream);
/* out[r] = table[ids[r]] (launchEmbeddingBatch, kernels.cuh:19-26). */
kimkv_status kimkv_model_embed(const uint16_t* table, const uint32_t* device_ids, uint32_t rows, uint32_t hidden,
                               uint16_t* out, kimkv_stream_t stream);
/* RMSNorm (launchRmsNormBatch, kernels.cuh:37-45): out[r] = x[src] * rsqrt(mean(x[src]^2) + eps) * weight,
 * src = device_rows ? device_rows[r] : r (row selection for the last position of each request). */
kimkv_status kimkv_model_rmsnorm(const uint16_t* x, const uint32_t* device_rows, uint32_t rows, const uint16_t* weight,
                                 uint32_t hidden, float eps, uint16_t* out, kimkv_stream_t stream);
/* RoPE (launchRopeBatch, kernels.cuh:58-68) fused with the q / k / v split of a
 * [rows][(QH + 2 KVH) * D] projection: q_out [rows][QH*D] and k_out
 * [rows][KVH*D] rotated by positions[r] (pairs (d, d + D/2), angle =
 * pos * theta^(-2d/D)), v_out [rows][KVH*D] copied. */
kimkv_status kimkv_model_rope_split(const uint16_t* qkv, const uint32_t* device_positions, uint32_t rows,
                                    uint32_t query_heads, uint32_t kv_heads, uint32_t head_dim, float theta,
                                    uint16_t* q_out, uint16_t* k_out, uint16_t* v_out, kimkv_stream_t stream);
/* SwiGLU (launchSwiGluBatch, kernels.cuh:95-102) of a fused [rows][2*inter]
 * gate|up projection: out[r][i] = silu(gate) * up. */
kimkv_status kimkv_model_swiglu(const uint16_t* gate_up, uint32_t rows, uint32_t intermediate, uint16_t* out,
                                kimkv_stream_t stream);
/* First index of each row's maximum (launchArgmaxBatch, kernels.cuh:111-117). */
kimkv_status kimkv_model_argmax(const float* logits, uint32_t rows, uint32_t vocabulary, uint32_t* device_out,
                                kimkv_stream_t stream);
/* Seeded weights: out[i] = fp16(float(synth(seed, row0 + i / cols, i % cols)) * scale). */
kimkv_status kimkv_fill_rows_scaled(uint16_t* device_out, uint64_t count, uint64_t seed, uint64_t row0, uint32_t cols,
                                    float scale, kimkv_stream_t stream);
/* out[i] = bits. */
kimkv_status kimkv_fill_f16(uint16_t* device_out, uint64_t count, uint16_t bits, kimkv_stream_t stream);

/* ---- synthetic inputs (benchmarks and tests) ----------------------------- */

/* Deterministic pseudo-normal fp16 value used for every synthetic tensor:
 *   h = mix64(mix64(seed + row * 0x9E3779B97F4A7C15) + col)
 *   v = (sum of the four 16-bit fields of h) - 131070          (Irwin-Hall n=4)
 *   x = fp16_rne(v * 2^-15)                                    (std ~1.155)
 * mix64 is the splitmix64 finalizer.  Host and device compute it bit-exactly. */
uint16_t kimkv_synth_value(uint64_t seed, uint64_t row, uint32_t col);

/* Row id of KV element (stream, layer, component, token). */
uint64_t kimkv_synth_kv_row(uint32_t stream, uint32_t layer, uint32_t component, uint32_t token);

/* Fills `count` fp16 values: out[i] = synth(seed, row0 + i / cols, i % cols). */
kimkv_status kimkv_fill_rows(uint16_t* device_out, uint64_t count, uint64_t seed,
                             uint64_t row0, uint32_t cols, kimkv_stream_t stream);

/* Fills a contiguous K/V block [layers][2][tokens][cols] (the layout of a
 * bulk append input): element (l, c, t, col) = synth(seed,
 * synth_kv_row(stream_id, l, c, token0 + t), col). */
kimkv_status kimkv_fill_kv(uint16_t* device_out, uint32_t layers, uint32_t tokens, uint32_t cols, uint64_t seed,
                           uint32_t stream_id, uint32_t token0, kimkv_stream_t stream);

/* Writes synthetic K/V for logical tokens [token_begin, token_end) of a table
 * straight into its pages: value(layer, comp, token, head, dim) =
 * synth(seed, kv_row(stream_id, layer, comp, token), head*D + dim).  Used to
 * materialise large contexts without host copies. */
kimkv_status kimkv_fill_table(const kimkv_storage* storage,
                              const kimkv_block_desc* device_descriptors, uint32_t descriptor_count,
                              uint32_t token_begin, uint32_t token_end,
                              uint64_t seed, uint32_t stream_id, kimkv_stream_t stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* KIMKV_HIP_H */
