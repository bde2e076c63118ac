"""ctypes binding of the host facade (include/kimkv_host.h, libkimkv.so).

Engine (EngineKvBackend + TokenTransaction), Cache (the CudaKvCache
counterpart) and Manager (KvCacheManager) for Python callers: tests and the
benchmark drive the C++ host layer through these.  Fails loudly when the
library has not been built.
"""
from __future__ import annotations

import ctypes
import os
from typing import List, Optional, Sequence

from . import device

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "_lib", "libkimkv.so")

U16, U32, U64, P, I = ctypes.c_uint16, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int

# EngineKvError values (include/kim-kv/engine/engine_kv.h).
ENGINE_ERRORS = ["none", "invalid_argument", "invalid_state", "request_not_found", "request_already_exists",
                 "request_conflict", "resource_exhausted", "layer_out_of_order", "submission_failed",
                 "execution_failed", "internal_error"]
# KvCacheError values (include/kim-kv/core/page_state.h).
KV_ERRORS = ["none", "invalid_argument", "request_not_found", "request_already_exists", "request_conflict",
             "resource_exhausted", "invalid_state", "token_reservation_not_found", "promotion_not_eligible",
             "promotion_not_found", "promotion_conflict", "internal_invariant_violation"]
PHASES = ["empty", "awaiting_layer_write", "awaiting_layer_attention", "ready_to_commit", "failed", "committed",
          "rolled_back"]


class MappingEntry(ctypes.Structure):
    _fields_ = [("logical_token_begin", U32), ("valid_tokens", U16), ("kind", ctypes.c_uint8),
                ("reserved", ctypes.c_uint8), ("slot", U32), ("generation", U32)]


class EngineConfig(ctypes.Structure):
    _fields_ = [("layers", U32), ("kv_heads", U32), ("head_dim", U32), ("query_heads", U32),
                ("attention_workspace_bytes", U64)]


class DecodeRequest(ctypes.Structure):
    _fields_ = [("layer", U32), ("reserved", U32), ("query", P), ("output", P), ("workspace", P),
                ("workspace_bytes", U64), ("attention_scale", ctypes.c_float)]


class EngineSnapshot(ctypes.Structure):
    _fields_ = [("request_count", U64), ("active_transaction_count", U64), ("committed_token_count", U64),
                ("batched_attention_submissions", U64), ("batched_attention_lanes", U64),
                ("batched_write_submissions", U64), ("primary_page_tokens", U32), ("secondary_page_tokens", U32),
                ("primary_page_capacity", U32), ("secondary_page_capacity", U32),
                ("allocated_primary_pages", U32), ("allocated_secondary_pages", U32),
                ("successful_primary_allocations", U64), ("successful_secondary_allocations", U64),
                ("failed_primary_allocations", U64), ("failed_secondary_allocations", U64),
                ("storage_reserved_bytes", U64)]


class PoolSnapshot(ctypes.Structure):
    _fields_ = [("kind", U32), ("total_slots", U32), ("free_slots", U32), ("allocated_slots", U32),
                ("successful_allocations", U64), ("successful_releases", U64), ("failed_allocations", U64),
                ("rejected_releases", U64)]


class ManagerSnapshot(ctypes.Structure):
    _fields_ = [("request_count", U64), ("promotion_count", U64), ("page_lease_count", U64),
                ("token_reservation_count", U64), ("micro_pool", PoolSnapshot), ("extent_pool", PoolSnapshot)]


class ModelConfig(ctypes.Structure):
    _fields_ = [("hidden_size", U32), ("intermediate_size", U32), ("layer_count", U32),
                ("attention_head_count", U32), ("kv_head_count", U32), ("head_dimension", U32),
                ("vocabulary_size", U32), ("max_position_embeddings", U32), ("bos_token_id", U32),
                ("eos_token_id", U32), ("rms_norm_epsilon", ctypes.c_float), ("rope_theta", ctypes.c_float)]


class SchedulerConfig(ctypes.Structure):
    _fields_ = [("max_active_requests", U32), ("max_batched_tokens", U32), ("max_kv_tokens", U64),
                ("prefill_chunk_size", U32)]


class IterationResult(ctypes.Structure):
    _fields_ = [("iteration", U64), ("model_forward_tokens", U32), ("model_forward_batches", U32),
                ("prefill_tokens", U32), ("decode_tokens", U32), ("terminals_produced", U32)]


class TerminalInfo(ctypes.Structure):
    _fields_ = [("request_id", U64), ("reason", U32), ("error", U32), ("prompt_tokens", U32),
                ("completion_tokens", U32), ("ttft_ns", U64), ("tpot_ns", U64), ("e2e_ns", U64)]


# GenerationTerminalReason / GenerationError / SchedulerAdmissionError (include/kim-kv/engine/*.h).
TERMINAL_REASONS = ["eos_token", "max_new_tokens", "cancelled", "runtime_stopped", "failed"]
GENERATION_ERRORS = ["none", "invalid_argument", "runtime_stopped", "model_failed", "kv_backend_failed",
                     "internal_error"]
ADMISSION_ERRORS = ["none", "invalid_argument", "runtime_stopped", "duplicate_request", "max_active_requests",
                    "kv_token_budget", "internal_error"]


class CacheResult(ctypes.Structure):
    _fields_ = [("metadata_error", I), ("device_status", I)]

    def ok(self) -> bool:
        return self.metadata_error == 0 and self.device_status == 0


_lib: Optional[ctypes.CDLL] = None

_SIG = {
    "kimkv_engine_create": (P, [ctypes.POINTER(EngineConfig), U32, U32]),
    "kimkv_engine_destroy": (None, [P]),
    "kimkv_engine_create_request": (I, [P, U64]),
    "kimkv_engine_fork_request": (I, [P, U64, U64]),
    "kimkv_engine_release_request": (I, [P, U64]),
    "kimkv_engine_reserve_token": (I, [P, U64, U32, P, ctypes.POINTER(P)]),
    "kimkv_engine_get_snapshot": (None, [P, ctypes.POINTER(EngineSnapshot)]),
    "kimkv_engine_check_invariants": (I, [P]),
    "kimkv_engine_inject_failure_once": (I, [P, U32]),
    "kimkv_engine_promote_request": (I, [P, U64, P, ctypes.POINTER(U32)]),
    "kimkv_engine_block_table": (I, [P, U64, ctypes.POINTER(U64), P, U32, ctypes.POINTER(U32)]),
    "kimkv_engine_storage": (P, [P]),
    "kimkv_engine_lane_record_launches": (U64, [P]),
    "kimkv_engine_append_prefill": (I, [P, U64, U32, P, P, I, ctypes.POINTER(U32)]),
    "kimkv_engine_permute_free_slots": (I, [P, U32, U64]),
    "kimkv_engine_reserve_batch": (None, [P, P, P, U32, P, P, P]),
    "kimkv_txn_commit_batch": (None, [P, U32, P]),
    "kimkv_txn_write_layer": (I, [P, U32, P, P]),
    "kimkv_txn_attend_layer": (I, [P, ctypes.POINTER(DecodeRequest)]),
    "kimkv_txn_commit": (I, [P]),
    "kimkv_txn_rollback": (I, [P]),
    "kimkv_txn_state": (None, [P, ctypes.POINTER(U32), ctypes.POINTER(U32), ctypes.POINTER(U32)]),
    "kimkv_txn_destroy": (None, [P]),
    "kimkv_attend_layer_batch": (None, [ctypes.POINTER(P), ctypes.POINTER(DecodeRequest), U32, P, U32,
                                        ctypes.POINTER(I)]),
    "kimkv_write_layer_batch": (None, [ctypes.POINTER(P), ctypes.POINTER(U32), ctypes.POINTER(P), ctypes.POINTER(P),
                                       U32, ctypes.POINTER(I)]),
    "kimkv_engine_prefill_begin": (I, [P, U64, U32, U32, P, ctypes.POINTER(P)]),
    "kimkv_prefill_write_layer": (I, [P, U32, P, P]),
    "kimkv_prefill_attend_layer": (I, [P, U32, P, P, ctypes.c_float]),
    "kimkv_prefill_finish": (I, [P]),
    "kimkv_prefill_destroy": (None, [P]),
    "kimkv_prefill_write_batch": (None, [ctypes.POINTER(P), U32, U32, ctypes.POINTER(P), ctypes.POINTER(P),
                                         ctypes.POINTER(I)]),
    "kimkv_prefill_attend_batch": (None, [ctypes.POINTER(P), U32, U32, ctypes.POINTER(P), ctypes.POINTER(P),
                                          ctypes.c_float, ctypes.POINTER(I)]),
    "kimkv_runner_create": (P, [P, ctypes.POINTER(ModelConfig), U64, U32, U32, P]),
    "kimkv_runner_create_from_archive": (P, [P, ctypes.c_char_p, ctypes.c_char_p, U32, U32, P, ctypes.c_char_p,
                                             ctypes.c_size_t]),
    "kimkv_runner_destroy": (None, [P]),
    "kimkv_runner_weight_bytes": (U64, [P]),
    "kimkv_runner_forward": (I, [P, U32, P, P, P, P, P, P, P]),
    "kimkv_runner_watch_logits": (I, [P, U32, P, P, P, P]),
    "kimkv_scheduler_create": (P, [P, P, ctypes.POINTER(SchedulerConfig)]),
    "kimkv_scheduler_destroy": (None, [P]),
    "kimkv_scheduler_submit": (I, [P, U64, P, U32, U32, ctypes.c_int64]),
    "kimkv_scheduler_cancel": (I, [P, U64]),
    "kimkv_scheduler_run_iteration": (None, [P, ctypes.POINTER(IterationResult)]),
    "kimkv_scheduler_drain": (U32, [P]),
    "kimkv_scheduler_collect": (U32, [P]),
    "kimkv_scheduler_terminal": (I, [P, U32, ctypes.POINTER(TerminalInfo), P, U32]),
    "kimkv_scheduler_clear_terminals": (None, [P]),
    "kimkv_scheduler_idle": (I, [P]),
    "kimkv_cache_create": (P, [device.Layout, U32, U32]),
    "kimkv_cache_destroy": (None, [P]),
    "kimkv_cache_status": (I, [P]),
    "kimkv_cache_manager": (P, [P]),
    "kimkv_cache_storage": (P, [P]),
    "kimkv_cache_append": (CacheResult, [P, U64, U32, P, P]),
    "kimkv_cache_append_batch": (None, [P, P, U32, U32, P, P, P]),
    "kimkv_cache_promote": (CacheResult, [P, U64, U32, P]),
    "kimkv_cache_gather": (CacheResult, [P, U64, P, P]),
    "kimkv_cache_reference_attention": (CacheResult, [P, U64, P, P, P]),
    "kimkv_cache_inject_failure_once": (None, [P, U32]),
    "kimkv_manager_create": (P, [U32, U32]),
    "kimkv_manager_destroy": (None, [P]),
    "kimkv_manager_create_request": (I, [P, U64]),
    "kimkv_manager_append": (I, [P, U64, U32]),
    "kimkv_manager_prepare_promotion": (I, [P, U64, U32, ctypes.POINTER(U64), P, P]),
    "kimkv_manager_commit_promotion": (I, [P, U64]),
    "kimkv_manager_fork_request": (I, [P, U64, U64]),
    "kimkv_manager_block_table": (I, [P, U64, ctypes.POINTER(U64), P, U32, ctypes.POINTER(U32)]),
    "kimkv_manager_permute_free_slots": (I, [P, U32, U64]),
    "kimkv_manager_check_invariants": (I, [P]),
    "kimkv_manager_get_snapshot": (None, [P, ctypes.POINTER(ManagerSnapshot)]),
    "kimkv_manager_release_request": (I, [P, U64]),
    "kimkv_seeded_permutation": (None, [U64, U32, P]),
}


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        device.lib()   # libkimkv.so links libkimkv_hip.so
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIG.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def _table(getter, handle, rid):
    version, count = U64(), U32()
    rc = getter(handle, rid, ctypes.byref(version), None, 0, ctypes.byref(count))
    if rc != 0:
        return None
    buf = (MappingEntry * max(count.value, 1))()
    rc = getter(handle, rid, ctypes.byref(version), buf, count.value, ctypes.byref(count))
    assert rc == 0
    return version.value, [(e.logical_token_begin, e.valid_tokens, e.kind, e.slot, e.generation)
                           for e in buf[:count.value]]


def storage_info(handle: int) -> device.StorageInfo:
    info = device.StorageInfo()
    device.check(device.lib().kimkv_storage_query(ctypes.c_void_p(handle), ctypes.byref(info)), "storage_query")
    return info


def descriptors_from_entries(entries, micro_tokens: int = 8, extent_tokens: int = 64):
    import numpy as np
    out = np.zeros(len(entries), dtype=device.BLOCK_DESC)
    for i, (b, v, k, s, g) in enumerate(entries):
        out[i] = (s, g, b, v, micro_tokens if k == 0 else extent_tokens, k)
    return out


class Transaction:
    def __init__(self, handle: int):
        self.h = handle

    def write_layer(self, layer: int, key: int, value: int) -> int:
        return lib().kimkv_txn_write_layer(self.h, layer, key, value)

    def attend_layer(self, layer, query, output, workspace, workspace_bytes, scale) -> int:
        r = DecodeRequest(layer, 0, query, output, workspace, workspace_bytes, scale)
        return lib().kimkv_txn_attend_layer(self.h, ctypes.byref(r))

    def commit(self) -> int:
        return lib().kimkv_txn_commit(self.h)

    def rollback(self) -> int:
        return lib().kimkv_txn_rollback(self.h)

    def state(self):
        ph, nl, pos = U32(), U32(), U32()
        lib().kimkv_txn_state(self.h, ctypes.byref(ph), ctypes.byref(nl), ctypes.byref(pos))
        return PHASES[ph.value], nl.value, pos.value

    def close(self) -> None:
        if self.h:
            lib().kimkv_txn_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


DECODE_ITEM_BYTES = 56   # kimkv_decode_item / DevicePagedDecodeBatchItem


def attend_layer_batch(txns: Sequence[Transaction], requests: Sequence[tuple],
                       device_items: Optional[device.DeviceBuffer] = None) -> List[int]:
    """requests[i] = (layer, query, output, workspace, workspace_bytes, scale).
    device_items: caller-owned scratch of >= len(txns) items (allocated here when omitted)."""
    n = len(txns)
    hs = (P * n)(*[t.h for t in txns])
    rs = (DecodeRequest * n)(*[DecodeRequest(r[0], 0, *r[1:]) for r in requests])
    st = (I * n)()
    scratch = device_items if device_items is not None else device.DeviceBuffer(n * DECODE_ITEM_BYTES)
    lib().kimkv_attend_layer_batch(hs, rs, n, scratch.ptr, scratch.nbytes // DECODE_ITEM_BYTES, st)
    if device_items is None:
        device.sync()
    return list(st)


def write_layer_batch(txns: Sequence[Transaction], layers, keys, values) -> List[int]:
    n = len(txns)
    hs = (P * n)(*[t.h for t in txns])
    st = (I * n)()
    lib().kimkv_write_layer_batch(hs, (U32 * n)(*layers), (P * n)(*keys), (P * n)(*values), n, st)
    return list(st)


class PrefillChunk:
    """A multi-token prompt chunk of one request (kimkv_engine_prefill_begin)."""

    def __init__(self, handle: int, begin: int, count: int):
        self.h, self.begin, self.count = handle, begin, count

    def write_layer(self, layer: int, key: int, value: int) -> int:
        return lib().kimkv_prefill_write_layer(self.h, layer, key, value)

    def attend_layer(self, layer: int, query: int, output: int, scale: float) -> int:
        return lib().kimkv_prefill_attend_layer(self.h, layer, query, output, scale)

    def finish(self) -> int:
        return lib().kimkv_prefill_finish(self.h)

    def close(self) -> None:
        if self.h:
            lib().kimkv_prefill_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def prefill_write_batch(chunks: Sequence[PrefillChunk], layer: int, keys, values) -> List[int]:
    n = len(chunks)
    st = (I * n)()
    lib().kimkv_prefill_write_batch((P * n)(*[c.h for c in chunks]), n, layer, (P * n)(*keys), (P * n)(*values), st)
    return list(st)


def prefill_attend_batch(chunks: Sequence[PrefillChunk], layer: int, queries, outputs, scale: float) -> List[int]:
    n = len(chunks)
    st = (I * n)()
    lib().kimkv_prefill_attend_batch((P * n)(*[c.h for c in chunks]), n, layer, (P * n)(*queries),
                                     (P * n)(*outputs), scale, st)
    return list(st)


class Engine:
    """createHeterogeneousHipEngineKvBackend through the C facade."""

    def __init__(self, layers, kv_heads, head_dim, query_heads, workspace_bytes, micro_capacity, extent_capacity):
        cfg = EngineConfig(layers, kv_heads, head_dim, query_heads, workspace_bytes)
        self.h = lib().kimkv_engine_create(ctypes.byref(cfg), micro_capacity, extent_capacity)
        if not self.h:
            raise RuntimeError("engine backend creation failed")
        self.layers, self.kv_heads, self.head_dim, self.query_heads = layers, kv_heads, head_dim, query_heads

    def create_request(self, rid) -> int:
        return lib().kimkv_engine_create_request(self.h, rid)

    def fork_request(self, src, child) -> int:
        return lib().kimkv_engine_fork_request(self.h, src, child)

    def release_request(self, rid) -> int:
        return lib().kimkv_engine_release_request(self.h, rid)

    def reserve_token(self, rid, expected, stream: Optional[device.Stream] = None):
        out = P()
        rc = lib().kimkv_engine_reserve_token(self.h, rid, expected, stream.handle if stream else None,
                                              ctypes.byref(out))
        return rc, (Transaction(out.value) if rc == 0 else None)

    def snapshot(self) -> EngineSnapshot:
        s = EngineSnapshot()
        lib().kimkv_engine_get_snapshot(self.h, ctypes.byref(s))
        return s

    def prefill_begin(self, rid, expected, token_count, stream: Optional[device.Stream] = None):
        out = P()
        rc = lib().kimkv_engine_prefill_begin(self.h, rid, expected, token_count,
                                              stream.handle if stream else None, ctypes.byref(out))
        return rc, (PrefillChunk(out.value, expected, token_count) if rc == 0 else None)

    def append_prefill(self, rid, token_count, device_kv, stream: Optional[device.Stream] = None, promote=True):
        n = U32()
        rc = lib().kimkv_engine_append_prefill(self.h, rid, token_count, device_kv,
                                               stream.handle if stream else None, 1 if promote else 0,
                                               ctypes.byref(n))
        return rc, n.value

    def permute_free_slots(self, kind: int, seed: int) -> int:
        return lib().kimkv_engine_permute_free_slots(self.h, kind, seed)

    def check_invariants(self) -> bool:
        return lib().kimkv_engine_check_invariants(self.h) == 1

    def inject_failure_once(self, point: str) -> bool:
        return lib().kimkv_engine_inject_failure_once(self.h, 0 if point == "submission" else 1) == 1

    def promote_request(self, rid, stream: Optional[device.Stream] = None):
        n = U32()
        rc = lib().kimkv_engine_promote_request(self.h, rid, stream.handle if stream else None, ctypes.byref(n))
        return rc, n.value

    def block_table(self, rid):
        return _table(lib().kimkv_engine_block_table, self.h, rid)

    def storage_handle(self) -> int:
        return lib().kimkv_engine_storage(self.h)

    def lane_record_launches(self) -> int:
        """Batched attention launches made from device lane records (evenly spaced lanes, at most 64)."""
        return int(lib().kimkv_engine_lane_record_launches(self.h))

    def close(self):
        if self.h:
            lib().kimkv_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Cache:
    """The CudaKvCache counterpart (HipKvCache)."""

    def __init__(self, layers, kv_heads, head_dim, micro_capacity, extent_capacity):
        self.h = lib().kimkv_cache_create(device.Layout(layers, kv_heads, head_dim), micro_capacity, extent_capacity)
        if not self.h:
            raise RuntimeError("cache creation failed")
        self.mgr = lib().kimkv_cache_manager(self.h)
        self.layers, self.kv_heads, self.head_dim = layers, kv_heads, head_dim

    def status(self) -> int:
        return lib().kimkv_cache_status(self.h)

    def create_request(self, rid) -> int:
        return lib().kimkv_manager_create_request(self.mgr, rid)

    def fork_request(self, src, child) -> int:
        return lib().kimkv_manager_fork_request(self.mgr, src, child)

    def append(self, rid, n, input_ptr, stream: Optional[device.Stream] = None) -> CacheResult:
        return lib().kimkv_cache_append(self.h, rid, n, input_ptr, stream.handle if stream else None)

    def append_batch(self, ids_array, token_count, inputs_array, results_array,
                     stream: Optional[device.Stream] = None) -> None:
        """ids_array: uint64[n]; inputs_array: uint64[n] device addresses; results_array:
        (CacheResult * n) receiving each request's result."""
        lib().kimkv_cache_append_batch(self.h, ids_array.ctypes.data_as(ctypes.c_void_p), len(ids_array),
                                       token_count, inputs_array.ctypes.data_as(ctypes.c_void_p),
                                       stream.handle if stream else None, results_array)

    def permute_free_slots(self, kind: int, seed: int) -> int:
        return lib().kimkv_manager_permute_free_slots(self.mgr, kind, seed)

    def promote(self, rid, begin, stream: Optional[device.Stream] = None) -> CacheResult:
        return lib().kimkv_cache_promote(self.h, rid, begin, stream.handle if stream else None)

    def gather(self, rid, out_ptr, stream: Optional[device.Stream] = None) -> CacheResult:
        return lib().kimkv_cache_gather(self.h, rid, out_ptr, stream.handle if stream else None)

    def reference_attention(self, rid, q_ptr, o_ptr, stream: Optional[device.Stream] = None) -> CacheResult:
        return lib().kimkv_cache_reference_attention(self.h, rid, q_ptr, o_ptr, stream.handle if stream else None)

    def inject_failure_once(self, point: str) -> None:
        lib().kimkv_cache_inject_failure_once(self.h, 0 if point == "submission" else 1)

    def storage_info(self) -> device.StorageInfo:
        return storage_info(lib().kimkv_cache_storage(self.h))

    def snapshot(self):
        s = ManagerSnapshot()
        lib().kimkv_manager_get_snapshot(self.mgr, ctypes.byref(s))
        return s

    def release_request(self, rid) -> int:
        return lib().kimkv_manager_release_request(self.mgr, rid)

    def block_table(self, rid):
        return _table(lib().kimkv_manager_block_table, self.mgr, rid)

    def check_invariants(self) -> bool:
        return lib().kimkv_manager_check_invariants(self.mgr) == 1

    def close(self):
        if self.h:
            lib().kimkv_cache_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


DECODE_REQUEST_DTYPE = None


def _request_dtype():
    import numpy as np
    global DECODE_REQUEST_DTYPE
    if DECODE_REQUEST_DTYPE is None:
        DECODE_REQUEST_DTYPE = np.dtype({
            "names": ["layer", "reserved", "query", "output", "workspace", "workspace_bytes", "attention_scale"],
            "formats": ["<u4", "<u4", "<u8", "<u8", "<u8", "<u8", "<f4"],
            "offsets": [0, 4, 8, 16, 24, 32, 40], "itemsize": ctypes.sizeof(DecodeRequest)})
    return DECODE_REQUEST_DTYPE


class LaneBatch:
    """Prebuilt argument arrays for driving the lanes through
    reserve -> per layer (writeLayerBatch, attendLayerBatch) -> commit with a
    constant number of FFI crossings per step.  keys/values/queries/outputs
    are [layers][lanes] device addresses (numpy views, updatable in place);
    the caller owns the buffers."""

    def __init__(self, engine: Engine, request_ids, workspaces, workspace_bytes: int, scale: float,
                 stream: Optional[device.Stream] = None):
        import numpy as np
        n = len(request_ids)
        L = engine.layers
        self.engine, self.n, self.L = engine, n, L
        self.stream = stream.handle if stream else None
        self.ids = np.ascontiguousarray(request_ids, dtype=np.uint64)
        self.expected = np.zeros(n, dtype=np.uint32)
        self.txns = np.zeros(n, dtype=np.uint64)
        self.status = np.zeros(n, dtype=np.int32)
        self.keys = np.zeros((L, n), dtype=np.uint64)
        self.values = np.zeros((L, n), dtype=np.uint64)
        self.layer_ids = np.repeat(np.arange(L, dtype=np.uint32)[:, None], n, axis=1)
        self._req = (DecodeRequest * (L * n))()
        self.requests = np.frombuffer(self._req, dtype=_request_dtype()).reshape(L, n)
        self.requests["layer"] = np.arange(L, dtype=np.uint32)[:, None]
        self.requests["workspace"] = np.asarray(workspaces, dtype=np.uint64)[None, :]
        self.requests["workspace_bytes"] = workspace_bytes
        self.requests["attention_scale"] = scale
        self._req_base = ctypes.addressof(self._req)
        self._req_stride = n * ctypes.sizeof(DecodeRequest)
        self.device_items = device.DeviceBuffer(n * DECODE_ITEM_BYTES)

    @property
    def queries(self):
        return self.requests["query"]

    @property
    def outputs(self):
        return self.requests["output"]

    @staticmethod
    def _p(a):
        return a.ctypes.data_as(ctypes.c_void_p)

    def _bind(self):
        """Argument pointers, built once (the arrays are updated in place)."""
        if getattr(self, "_args", None) is None:
            P_ = ctypes.POINTER(P)
            self._args = {
                "txns": ctypes.cast(self._p(self.txns), P_),
                "status": ctypes.cast(self._p(self.status), ctypes.POINTER(I)),
                "layers": [ctypes.cast(self._p(self.layer_ids[l]), ctypes.POINTER(U32)) for l in range(self.L)],
                "keys": [ctypes.cast(self._p(self.keys[l]), P_) for l in range(self.L)],
                "values": [ctypes.cast(self._p(self.values[l]), P_) for l in range(self.L)],
                "reqs": [ctypes.cast(ctypes.c_void_p(self._req_base + l * self._req_stride),
                                     ctypes.POINTER(DecodeRequest)) for l in range(self.L)],
                "ids": self._p(self.ids), "expected": self._p(self.expected),
                "txns_v": self._p(self.txns), "status_v": self._p(self.status),
            }
        return self._args

    def reserve(self, expected) -> None:
        a = self._bind()
        self.expected[:] = expected
        lib().kimkv_engine_reserve_batch(self.engine.h, a["ids"], a["expected"], self.n, self.stream, a["txns_v"],
                                         a["status_v"])

    def write(self, layer: int) -> None:
        a = self._bind()
        lib().kimkv_write_layer_batch(a["txns"], a["layers"][layer], a["keys"][layer], a["values"][layer], self.n,
                                      a["status"])

    def attend(self, layer: int) -> None:
        a = self._bind()
        lib().kimkv_attend_layer_batch(a["txns"], a["reqs"][layer], self.n, self.device_items.ptr, self.n,
                                       a["status"])

    def commit(self) -> None:
        a = self._bind()
        lib().kimkv_txn_commit_batch(a["txns_v"], self.n, a["status_v"])

    def failed(self) -> bool:
        return bool(self.status.any())


class Runner:
    """HipTinyLlamaRunner on an Engine: seeded N(0, 0.02) fp16 weights, or a
    checkpoint archive (Runner.from_archive)."""

    def __init__(self, engine: "Engine", model: ModelConfig, seed: int, max_positions: int, max_spans: int,
                 stream: Optional[device.Stream] = None):
        self.engine, self.model = engine, model
        self.h = lib().kimkv_runner_create(engine.h, ctypes.byref(model), seed, max_positions, max_spans,
                                           stream.handle if stream else None)
        if not self.h:
            raise RuntimeError("model runner creation failed")

    @classmethod
    def from_archive(cls, engine: "Engine", model: ModelConfig, manifest_path: str, data_path: str,
                     max_positions: int, max_spans: int, stream: Optional[device.Stream] = None) -> "Runner":
        """Weights from a weight manifest + fp16 data file (model: the manifest's dimensions, for the caller's
        bookkeeping; the library takes them from the manifest).  Raises with the library's reason."""
        self = cls.__new__(cls)
        self.engine, self.model = engine, model
        reason = ctypes.create_string_buffer(512)
        self.h = lib().kimkv_runner_create_from_archive(engine.h, manifest_path.encode(), data_path.encode(),
                                                        max_positions, max_spans, stream.handle if stream else None,
                                                        reason, len(reason))
        if not self.h:
            raise RuntimeError("model runner creation failed: " + reason.value.decode())
        return self

    def weight_bytes(self) -> int:
        return lib().kimkv_runner_weight_bytes(self.h)

    def watch_logits(self, request_ids):
        """kimkv_runner_watch_logits: returns (rows [n][vocabulary] fp32, positions [n], counts [n]), filled
        after every forward that holds a span of request_ids[k]; watch_logits([]) ends the watch."""
        import numpy as np
        ids = np.ascontiguousarray(np.asarray(request_ids, dtype=np.uint64))
        n = ids.size
        rows = np.zeros((max(n, 1), self.model.vocabulary_size), dtype=np.float32)
        positions = np.zeros(max(n, 1), dtype=np.uint32)
        counts = np.zeros(max(n, 1), dtype=np.uint32)
        self._watch = (ids, rows, positions, counts)     # kept alive while the library writes them
        rc = lib().kimkv_runner_watch_logits(self.h, n, ids.ctypes.data if n else None, rows.ctypes.data,
                                             positions.ctypes.data, counts.ctypes.data)
        if rc != 0:
            raise RuntimeError("watch_logits failed")
        return rows[:n], positions[:n], counts[:n]

    def forward(self, spans, want_logits: bool = False):
        """spans: list of (request_id, first_position, [token ids]).  Returns
        (next_tokens, step_ok, logits or None)."""
        import numpy as np
        n = len(spans)
        ids = np.array([s[0] for s in spans], dtype=np.uint64)
        first = np.array([s[1] for s in spans], dtype=np.uint32)
        counts = np.array([len(s[2]) for s in spans], dtype=np.uint32)
        tokens = np.concatenate([np.asarray(s[2], dtype=np.uint32) for s in spans])
        nxt = np.zeros(n, dtype=np.uint32)
        ok = np.zeros(n, dtype=np.int32)
        logits = np.zeros((n, self.model.vocabulary_size), dtype=np.float32) if want_logits else None
        rc = lib().kimkv_runner_forward(self.h, n, ids.ctypes.data, first.ctypes.data, counts.ctypes.data,
                                        tokens.ctypes.data, nxt.ctypes.data, ok.ctypes.data,
                                        logits.ctypes.data if logits is not None else None)
        if rc != 0:
            raise RuntimeError("model forward failed")
        return nxt, ok.astype(bool), logits

    def close(self):
        if self.h:
            lib().kimkv_runner_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Scheduler:
    """IterationSchedulerRuntime over an Engine and a Runner."""

    def __init__(self, engine: "Engine", runner: Runner, max_active: int, max_batched_tokens: int,
                 max_kv_tokens: int, prefill_chunk: int):
        self.engine, self.runner = engine, runner
        cfg = SchedulerConfig(max_active, max_batched_tokens, max_kv_tokens, prefill_chunk)
        self.h = lib().kimkv_scheduler_create(engine.h, runner.h, ctypes.byref(cfg))
        if not self.h:
            raise RuntimeError("scheduler creation failed")

    def submit(self, rid: int, prompt, max_new_tokens: int, eos: int = -1) -> str:
        import numpy as np
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.uint32))
        rc = lib().kimkv_scheduler_submit(self.h, rid, p.ctypes.data if p.size else None, p.size, max_new_tokens, eos)
        return ADMISSION_ERRORS[rc]

    def cancel(self, rid: int) -> bool:
        return lib().kimkv_scheduler_cancel(self.h, rid) == 1

    def run_iteration(self) -> IterationResult:
        r = IterationResult()
        lib().kimkv_scheduler_run_iteration(self.h, ctypes.byref(r))
        return r

    def idle(self) -> bool:
        return lib().kimkv_scheduler_idle(self.h) == 1

    def _take(self, count: int):
        out = []
        for i in range(count):
            info = TerminalInfo()
            n = lib().kimkv_scheduler_terminal(self.h, i, ctypes.byref(info), None, 0)
            toks = (U32 * max(n, 1))()
            lib().kimkv_scheduler_terminal(self.h, i, ctypes.byref(info), toks, n)
            out.append({"request_id": info.request_id, "reason": TERMINAL_REASONS[info.reason],
                        "error": GENERATION_ERRORS[info.error], "prompt_tokens": info.prompt_tokens,
                        "completion_tokens": info.completion_tokens, "tokens": list(toks[:n]),
                        "ttft_ns": info.ttft_ns, "tpot_ns": info.tpot_ns, "e2e_ns": info.e2e_ns})
        lib().kimkv_scheduler_clear_terminals(self.h)
        return out

    def drain(self):
        return self._take(lib().kimkv_scheduler_drain(self.h))

    def take_terminals(self):
        return self._take(lib().kimkv_scheduler_collect(self.h))

    def close(self):
        if self.h:
            lib().kimkv_scheduler_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
