/*
 * kimkv_host.h -- C facade of the C++ host layer (libkimkv.so).
 *
 * The C++ API under include/kim-kv/ mirrors the reference's include/kim-kv
 * (same class names, arguments and error enums).  This header flattens the
 * parts a non-C++ caller binds (ctypes, cgo, JNI) into plain functions.
 * Return codes are the numeric values of the C++ enums:
 *   KvCacheError   (include/kim-kv/core/page_state.h:67-80)   for kimkv_manager_*
 *   EngineKvError  (include/kim-kv/engine/engine_kv.h:25-37)  for kimkv_engine_* / kimkv_txn_*
 *   KvCacheError + kimkv_status pair for kimkv_cache_* (CudaKvOperationResult,
 *   include/kim-kv/cuda/cuda_kv_cache.h:16-31).
 */
#ifndef KIMKV_HOST_H
#define KIMKV_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "kimkv_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* MappingEntry (include/kim-kv/core/block_table.h:13-41), flattened. */
typedef struct kimkv_mapping_entry {
    uint32_t logical_token_begin;
    uint16_t valid_tokens;
    uint8_t kind;
    uint8_t reserved;
    uint32_t slot;
    uint32_t generation;
} kimkv_mapping_entry;

/* PageHandle (include/kim-kv/core/page_handle.h:10-47). */
typedef struct kimkv_page_handle {
    uint32_t kind;
    uint32_t slot;
    uint32_t generation;
} kimkv_page_handle;

/* PageMetadataSnapshot (include/kim-kv/runtime/kv_cache_manager.h:21-33). */
typedef struct kimkv_page_metadata {
    uint32_t state;          /* PageState: 0 free 1 mutable 2 sealed 3 copy_target 4 retiring */
    uint32_t valid_tokens;
    uint32_t ref_count;
    uint32_t promotion_pins;
    uint32_t inflight_readers;
    uint32_t reserved;
    uint64_t mutable_owner;
} kimkv_page_metadata;

/* PagePoolSnapshot (include/kim-kv/core/page_pool.h:25-40). */
typedef struct kimkv_pool_snapshot {
    uint32_t kind;
    uint32_t total_slots;
    uint32_t free_slots;
    uint32_t allocated_slots;
    uint64_t successful_allocations;
    uint64_t successful_releases;
    uint64_t failed_allocations;
    uint64_t rejected_releases;
} kimkv_pool_snapshot;

/* KvCacheManagerSnapshot (kv_cache_manager.h:35-42). */
typedef struct kimkv_manager_snapshot {
    uint64_t request_count;
    uint64_t promotion_count;
    uint64_t page_lease_count;
    uint64_t token_reservation_count;
    kimkv_pool_snapshot micro_pool;
    kimkv_pool_snapshot extent_pool;
} kimkv_manager_snapshot;

/* ---- KvCacheManager (include/kim-kv/runtime/kv_cache_manager.h:44-277) ---- */
typedef struct kimkv_manager kimkv_manager;

kimkv_manager* kimkv_manager_create(uint32_t micro_capacity, uint32_t extent_capacity);
void kimkv_manager_destroy(kimkv_manager* m);
int kimkv_manager_create_request(kimkv_manager* m, uint64_t request_id);
int kimkv_manager_append(kimkv_manager* m, uint64_t request_id, uint32_t token_count);
/* reserveToken; the reserved (candidate) table is copied out when entries != NULL. */
int kimkv_manager_reserve_token(kimkv_manager* m, uint64_t request_id, uint32_t expected_committed_tokens,
                                uint64_t* reservation_id, uint64_t* reserved_version,
                                kimkv_mapping_entry* entries, uint32_t capacity, uint32_t* count);
int kimkv_manager_commit_token(kimkv_manager* m, uint64_t reservation_id);
int kimkv_manager_rollback_token(kimkv_manager* m, uint64_t reservation_id);
int kimkv_manager_seal_tail(kimkv_manager* m, uint64_t request_id);
int kimkv_manager_fork_request(kimkv_manager* m, uint64_t source_request_id, uint64_t child_request_id);
int kimkv_manager_release_request(kimkv_manager* m, uint64_t request_id);
/* preparePromotion; sources[8] and target receive the handles when non-NULL. */
int kimkv_manager_prepare_promotion(kimkv_manager* m, uint64_t request_id, uint32_t logical_token_begin,
                                    uint64_t* promotion_id, kimkv_page_handle* sources,
                                    kimkv_page_handle* target);
int kimkv_manager_commit_promotion(kimkv_manager* m, uint64_t promotion_id);
int kimkv_manager_rollback_promotion(kimkv_manager* m, uint64_t promotion_id);
int kimkv_manager_acquire_request_lease(kimkv_manager* m, uint64_t request_id, uint64_t* lease_id);
int kimkv_manager_acquire_promotion_lease(kimkv_manager* m, uint64_t promotion_id, uint64_t* lease_id);
int kimkv_manager_acquire_reservation_lease(kimkv_manager* m, uint64_t reservation_id, uint64_t* lease_id);
int kimkv_manager_release_lease(kimkv_manager* m, uint64_t lease_id);
/* blockTable: returns 0, RequestNotFound (2), or InvalidArgument (1) when
 * `capacity` is too small (*count then holds the needed size). */
int kimkv_manager_block_table(const kimkv_manager* m, uint64_t request_id, uint64_t* version,
                              kimkv_mapping_entry* entries, uint32_t capacity, uint32_t* count);
/* pageMetadata: 0 when the handle names a live runtime slot, 1 otherwise. */
int kimkv_manager_page_metadata(const kimkv_manager* m, kimkv_page_handle handle, kimkv_page_metadata* out);
void kimkv_manager_get_snapshot(const kimkv_manager* m, kimkv_manager_snapshot* out);
int kimkv_manager_check_invariants(const kimkv_manager* m);

/* Seeded Fisher-Yates permutation of 0..n-1 driven by splitmix64 (shared by
 * the benchmark, the tests and the oracle's trace driver). */
void kimkv_seeded_permutation(uint64_t seed, uint32_t n, uint32_t* out);

/* Reorders a fresh manager's free lists through its public API only, so that
 * the next allocations of `kind` return slots perm(seed)[0], perm[1], ...:
 * every slot is allocated (one throw-away request per page, extents through
 * promotion) and the requests are released in reverse permutation order.
 * Slot generations advance by one.  Returns KvCacheError. */
int kimkv_manager_permute_free_slots(kimkv_manager* m, uint32_t kind, uint64_t seed);

/* ---- engine backend (include/kim-kv/engine/engine_kv.h:255-427) ----------- */
typedef struct kimkv_engine kimkv_engine;
typedef struct kimkv_txn kimkv_txn;

typedef struct kimkv_engine_config {
    uint32_t layers;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t query_heads;
    uint64_t attention_workspace_bytes;
} kimkv_engine_config;

/* PagedDecodeRequest (engine_kv.h:151-158). */
typedef struct kimkv_decode_request {
    uint32_t layer;
    uint32_t reserved;
    const uint16_t* query;
    uint16_t* output;
    void* workspace;
    uint64_t workspace_bytes;
    float attention_scale;
} kimkv_decode_request;

/* EngineKvBackendSnapshot (engine_kv.h:372-391). */
typedef struct kimkv_engine_snapshot {
    uint64_t request_count;
    uint64_t active_transaction_count;
    uint64_t committed_token_count;
    uint64_t batched_attention_submissions;
    uint64_t batched_attention_lanes;
    uint64_t batched_write_submissions;
    uint32_t primary_page_tokens;
    uint32_t secondary_page_tokens;
    uint32_t primary_page_capacity;
    uint32_t secondary_page_capacity;
    uint32_t allocated_primary_pages;
    uint32_t allocated_secondary_pages;
    uint64_t successful_primary_allocations;
    uint64_t successful_secondary_allocations;
    uint64_t failed_primary_allocations;
    uint64_t failed_secondary_allocations;
    uint64_t storage_reserved_bytes;
} kimkv_engine_snapshot;

/* createHeterogeneousCudaEngineKvBackend (include/kim-kv/cuda/cuda_engine_kv_backend.h:11-16). */
kimkv_engine* kimkv_engine_create(const kimkv_engine_config* config, uint32_t micro_capacity,
                                  uint32_t extent_capacity);
void kimkv_engine_destroy(kimkv_engine* e);
int kimkv_engine_create_request(kimkv_engine* e, uint64_t request_id);
int kimkv_engine_fork_request(kimkv_engine* e, uint64_t source_request_id, uint64_t child_request_id);
int kimkv_engine_release_request(kimkv_engine* e, uint64_t request_id);
/* reserveToken: *txn receives a transaction owned by the caller (kimkv_txn_destroy). */
int kimkv_engine_reserve_token(kimkv_engine* e, uint64_t request_id, uint32_t expected_committed_tokens,
                               kimkv_stream_t stream, kimkv_txn** txn);
void kimkv_engine_get_snapshot(const kimkv_engine* e, kimkv_engine_snapshot* out);
int kimkv_engine_check_invariants(const kimkv_engine* e);
/* injectCudaEngineFailureOnce (cuda_engine_kv_backend.h:25-29): point 0 = submission, 1 = completion. */
int kimkv_engine_inject_failure_once(kimkv_engine* e, uint32_t point);
/* Engine-path promotion (no reference counterpart: the reference engine never
 * promotes).  Promotes every eligible 8-micro run of a committed request on
 * `stream` and waits for it. */
int kimkv_engine_promote_request(kimkv_engine* e, uint64_t request_id, kimkv_stream_t stream,
                                 uint32_t* promoted);
/* Copies out a request's committed block table (same contract as kimkv_manager_block_table). */
int kimkv_engine_block_table(const kimkv_engine* e, uint64_t request_id, uint64_t* version,
                             kimkv_mapping_entry* entries, uint32_t capacity, uint32_t* count);
/* The engine's device storage (for data-path helpers such as kimkv_gather). */
const kimkv_storage* kimkv_engine_storage(const kimkv_engine* e);
/* Batched attention launches that read their lanes from device lane records
 * (kimkv_paged_decode_lanes) instead of items staged in host memory: batches
 * of at most 64 lanes whose queries, outputs, workspaces and new K/V rows are
 * evenly spaced.  No reference counterpart (a test hook for which path ran). */
uint64_t kimkv_engine_lane_record_launches(const kimkv_engine* e);
/* Bulk prompt append (no reference counterpart: the reference engine appends
 * one token per transaction).  device_kv is [layer][K/V][token_count][head][dim]
 * fp16; waits for the copy, seals a full tail and, when promote != 0,
 * promotes every complete 64-token run (count in *promoted).  A device
 * failure cancels the request. */
int kimkv_engine_append_prefill(kimkv_engine* e, uint64_t request_id, uint32_t token_count,
                                const uint16_t* device_kv, kimkv_stream_t stream, int promote, uint32_t* promoted);
/* Seeded permutation of a pool's free list (kind 0 micro, 1 extent) while the
 * engine has no request: page ids then come out scattered over the pool. */
int kimkv_engine_permute_free_slots(kimkv_engine* e, uint32_t kind, uint64_t seed);
/* reserveToken for `count` requests on one stream: txns[i] / statuses[i] as
 * kimkv_engine_reserve_token would return them one by one. */
void kimkv_engine_reserve_batch(kimkv_engine* e, const uint64_t* request_ids, const uint32_t* expected_committed,
                                uint32_t count, kimkv_stream_t stream, kimkv_txn** txns, int* statuses);

/* TokenTransaction (engine_kv.h:298-351). */
int kimkv_txn_write_layer(kimkv_txn* t, uint32_t layer, const uint16_t* key, const uint16_t* value);
int kimkv_txn_attend_layer(kimkv_txn* t, const kimkv_decode_request* request);
int kimkv_txn_commit(kimkv_txn* t);
int kimkv_txn_rollback(kimkv_txn* t);
/* Fills phase (TokenTransactionPhase), next layer and logical position. */
void kimkv_txn_state(const kimkv_txn* t, uint32_t* phase, uint32_t* next_layer, uint32_t* position);
void kimkv_txn_destroy(kimkv_txn* t);   /* rolls back when not committed */
/* commit of `count` transactions; each is destroyed afterwards and txns[i]
 * set to NULL (a failed commit has rolled back). */
void kimkv_txn_commit_batch(kimkv_txn** txns, uint32_t count, int* statuses);

/* attendLayerBatch (engine_kv.h:355): statuses[i] receives each lane's
 * EngineKvError.  device_items / device_capacity are PagedDecodeBatch's
 * caller-owned device scratch (capacity >= count is required, as in the
 * reference); the HIP backend stages the items together with the chunk
 * prefix through its own ring, so the scratch is never written. */
void kimkv_attend_layer_batch(kimkv_txn** txns, const kimkv_decode_request* requests, uint32_t count,
                              void* device_items, uint32_t device_capacity, int* statuses);
/* writeLayerBatch: batched form of TokenTransaction::writeLayer (one kernel for all lanes). */
void kimkv_write_layer_batch(kimkv_txn** txns, const uint32_t* layers, const uint16_t* const* keys,
                             const uint16_t* const* values, uint32_t count, int* statuses);

/* ---- chunked prefill (no reference counterpart: the reference advances a
 * prompt one position per token transaction) ------------------------------
 * kimkv_engine_prefill_begin appends token_count positions to a committed
 * request whose committed length is expected_committed_tokens and returns a
 * chunk handle.  Then, for layer 0, 1, ... in order: write the chunk's K/V
 * (each [token_count][kv_heads][head_dim] fp16, device memory), then attend
 * its queries ([token_count][query_heads][head_dim]) causally over the
 * request's tokens, output row i = decode of the first T0 + i + 1 tokens.
 * kimkv_prefill_finish waits for the chunk's work and commits the tokens; a
 * failure (or a chunk abandoned before its last layer) cancels the request.
 * While a chunk is open, the request refuses reservation, fork, promotion and
 * release (EngineKvError::InvalidState).  Calls only enqueue work on the
 * chunk's stream before finish. */
typedef struct kimkv_prefill_chunk kimkv_prefill_chunk;
int kimkv_engine_prefill_begin(kimkv_engine* e, uint64_t request_id, uint32_t expected_committed_tokens,
                               uint32_t token_count, kimkv_stream_t stream, kimkv_prefill_chunk** chunk);
int kimkv_prefill_write_layer(kimkv_prefill_chunk* c, uint32_t layer, const uint16_t* key, const uint16_t* value);
int kimkv_prefill_attend_layer(kimkv_prefill_chunk* c, uint32_t layer, const uint16_t* query, uint16_t* output,
                               float attention_scale);
int kimkv_prefill_finish(kimkv_prefill_chunk* c);
void kimkv_prefill_destroy(kimkv_prefill_chunk* c);   /* finishes first when still open */
/* One layer step of `count` chunks of one engine and stream: one append
 * launch (write) or one prefill-attention launch (attend) for all of them. */
void kimkv_prefill_write_batch(kimkv_prefill_chunk** chunks, uint32_t count, uint32_t layer,
                               const uint16_t* const* keys, const uint16_t* const* values, int* statuses);
void kimkv_prefill_attend_batch(kimkv_prefill_chunk** chunks, uint32_t count, uint32_t layer,
                                const uint16_t* const* queries, uint16_t* const* outputs, float attention_scale,
                                int* statuses);

/* ---- model runner and iteration scheduler ----------------------------------
 * HipTinyLlamaRunner (include/kim-kv/hip/hip_model_runner.h; counterpart of
 * createCudaTinyLlamaModelRunner, include/kim-kv/cuda/cuda_model_runner.h)
 * and IterationSchedulerRuntime (include/kim-kv/engine/iteration_scheduler.h:
 * 132-180) over an engine.  Weights are seeded N(0, 0.02) fp16. */
typedef struct kimkv_runner kimkv_runner;
typedef struct kimkv_scheduler kimkv_scheduler;

/* TinyLlamaConfig (include/kim-kv/model/tinyllama_config.h). */
typedef struct kimkv_model_config {
    uint32_t hidden_size;
    uint32_t intermediate_size;
    uint32_t layer_count;
    uint32_t attention_head_count;
    uint32_t kv_head_count;
    uint32_t head_dimension;
    uint32_t vocabulary_size;
    uint32_t max_position_embeddings;
    uint32_t bos_token_id;
    uint32_t eos_token_id;
    float rms_norm_epsilon;
    float rope_theta;
} kimkv_model_config;

/* NULL on a shape mismatch with the engine or an allocation failure. */
kimkv_runner* kimkv_runner_create(kimkv_engine* e, const kimkv_model_config* model, uint64_t weight_seed,
                                  uint32_t max_positions, uint32_t max_spans, kimkv_stream_t stream);
/* A runner whose weights come from a checkpoint archive: manifest_path is the
 * weight manifest (include/kim-kv/model/weight_manifest.h), data_path its
 * fp16 data file; the model dimensions are the manifest's.  On failure
 * returns NULL and writes a NUL-terminated reason into error (when
 * error_capacity > 0).  Counterpart of the reference's
 * createCudaTinyLlamaModelRunner(kv, manifest_path, data_path, ...)
 * (src/cuda/model/runner_factory.cpp:11-196). */
kimkv_runner* kimkv_runner_create_from_archive(kimkv_engine* e, const char* manifest_path, const char* data_path,
                                               uint32_t max_positions, uint32_t max_spans, kimkv_stream_t stream,
                                               char* error, size_t error_capacity);
void kimkv_runner_destroy(kimkv_runner* r);
uint64_t kimkv_runner_weight_bytes(const kimkv_runner* r);
/* One forward over span_count spans (span i: request_ids[i], positions
 * [first_positions[i], + token_counts[i]), its tokens next in `tokens`).
 * next_tokens[i] = greedy token after the span; step_ok[i] = 1 if the span
 * succeeded; logits (nullable) receives [span_count][vocabulary] fp32.
 * Returns 0 when the call ran (per-span failures in step_ok), else -1. */
int kimkv_runner_forward(kimkv_runner* r, uint32_t span_count, const uint64_t* request_ids,
                         const uint32_t* first_positions, const uint32_t* token_counts, const uint32_t* tokens,
                         uint32_t* next_tokens, int* step_ok, float* logits);

/* HipTinyLlamaRunner::watchLogits: after each forward (the scheduler's
 * included) holding a span of request_ids[k], the fp32 logits after that
 * span's last position go to rows + k * vocabulary, positions[k] gets that
 * position and counts[k] is incremented.  Host buffers owned by the caller,
 * valid while watched; count 0 ends the watch.  No counterpart in the
 * reference.  Returns 0, or -1 for a null argument. */
int kimkv_runner_watch_logits(kimkv_runner* r, uint32_t count, const uint64_t* request_ids, float* rows,
                              uint32_t* positions, uint32_t* counts);

/* IterationSchedulerConfig. */
typedef struct kimkv_scheduler_config {
    uint32_t max_active_requests;
    uint32_t max_batched_tokens;
    uint64_t max_kv_tokens;
    uint32_t prefill_chunk_size;
} kimkv_scheduler_config;

/* SchedulerIterationResult. */
typedef struct kimkv_iteration_result {
    uint64_t iteration;
    uint32_t model_forward_tokens;
    uint32_t model_forward_batches;
    uint32_t prefill_tokens;
    uint32_t decode_tokens;
    uint32_t terminals_produced;
} kimkv_iteration_result;

/* GenerationTerminal without its token list (kimkv_scheduler_terminal_tokens). */
typedef struct kimkv_terminal_info {
    uint64_t request_id;
    uint32_t reason;               /* GenerationTerminalReason */
    uint32_t error;                /* GenerationError */
    uint32_t prompt_tokens;
    uint32_t completion_tokens;
    uint64_t ttft_ns;
    uint64_t tpot_ns;
    uint64_t e2e_ns;
} kimkv_terminal_info;

kimkv_scheduler* kimkv_scheduler_create(kimkv_engine* e, kimkv_runner* r, const kimkv_scheduler_config* config);
void kimkv_scheduler_destroy(kimkv_scheduler* s);   /* stops and reclaims active requests */
/* submit(): returns SchedulerAdmissionError; eos_token_id < 0 = the model's EOS. */
int kimkv_scheduler_submit(kimkv_scheduler* s, uint64_t request_id, const uint32_t* prompt, uint32_t prompt_length,
                           uint32_t max_new_tokens, int64_t eos_token_id);
int kimkv_scheduler_cancel(kimkv_scheduler* s, uint64_t request_id);
void kimkv_scheduler_run_iteration(kimkv_scheduler* s, kimkv_iteration_result* out);
/* drain() / takeTerminals(): terminals move to the handle's delivery list;
 * both return the list's new length. */
uint32_t kimkv_scheduler_drain(kimkv_scheduler* s);
uint32_t kimkv_scheduler_collect(kimkv_scheduler* s);
/* Reads delivered terminal `index`; its tokens go to `tokens` (up to
 * capacity); returns the token count, or -1 for a bad index. */
int kimkv_scheduler_terminal(const kimkv_scheduler* s, uint32_t index, kimkv_terminal_info* info, uint32_t* tokens,
                             uint32_t capacity);
void kimkv_scheduler_clear_terminals(kimkv_scheduler* s);
int kimkv_scheduler_idle(const kimkv_scheduler* s);

/* ---- CudaKvCache equivalent (include/kim-kv/cuda/cuda_kv_cache.h:33-100) --- */
typedef struct kimkv_cache kimkv_cache;

typedef struct kimkv_cache_result {
    int metadata_error;     /* KvCacheError */
    int device_status;      /* kimkv_status */
} kimkv_cache_result;

kimkv_cache* kimkv_cache_create(kimkv_layout layout, uint32_t micro_capacity, uint32_t extent_capacity);
void kimkv_cache_destroy(kimkv_cache* c);
int kimkv_cache_status(const kimkv_cache* c);
kimkv_manager* kimkv_cache_manager(kimkv_cache* c);
const kimkv_storage* kimkv_cache_storage(const kimkv_cache* c);
/* append for `count` requests in one launch (HipKvCache::appendBatch; no
 * reference counterpart).  device_inputs[i] is request i's
 * [layer][K/V][token_count][head][dim] block; results[i] as kimkv_cache_append. */
void kimkv_cache_append_batch(kimkv_cache* c, const uint64_t* request_ids, uint32_t count, uint32_t token_count,
                              const uint16_t* const* device_inputs, kimkv_stream_t stream,
                              kimkv_cache_result* results);
kimkv_cache_result kimkv_cache_append(kimkv_cache* c, uint64_t request_id, uint32_t token_count,
                                      const uint16_t* device_input, kimkv_stream_t stream);
kimkv_cache_result kimkv_cache_promote(kimkv_cache* c, uint64_t request_id, uint32_t logical_token_begin,
                                       kimkv_stream_t stream);
kimkv_cache_result kimkv_cache_gather(kimkv_cache* c, uint64_t request_id, uint16_t* device_output,
                                      kimkv_stream_t stream);
kimkv_cache_result kimkv_cache_reference_attention(kimkv_cache* c, uint64_t request_id,
                                                   const float* device_query, float* device_output,
                                                   kimkv_stream_t stream);
void kimkv_cache_inject_failure_once(kimkv_cache* c, uint32_t point);

#ifdef __cplusplus
}
#endif

#endif /* KIMKV_HOST_H */
