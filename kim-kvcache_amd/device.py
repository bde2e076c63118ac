"""ctypes binding of the device C-ABI (include/kimkv_hip.h).

This is the Python-side binding a maintainer would add for the data path.
It loads the in-tree libkimkv_hip.so and fails loudly when it is missing:
there is no CPU fallback.  Device memory, streams and events come from the
library itself (numpy holds host data), so no second HIP runtime is loaded.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "_lib", "libkimkv_hip.so")

OK = 0
INVALID_ARGUMENT = 1
STATUS_NAMES = {
    0: "ok", 1: "invalid_argument", 2: "runtime_unavailable", 3: "allocation_failed",
    4: "submission_failed", 5: "not_ready", 6: "execution_failed", 7: "internal_error",
}
PAGE_MICRO = 0
PAGE_EXTENT = 1

# numpy views of the C structs (field order, offsets and sizes of kimkv_hip.h).
BLOCK_DESC = np.dtype({
    "names": ["slot", "generation", "logical_token_begin", "valid_tokens", "page_token_capacity", "kind"],
    "formats": ["<u4", "<u4", "<u4", "<u2", "<u2", "u1"],
    "offsets": [0, 4, 8, 12, 14, 16],
    "itemsize": 20,
})
DECODE_ITEM = np.dtype({
    "names": ["descriptors", "descriptor_count", "token_count", "layer", "query", "workspace", "output",
              "attention_scale"],
    "formats": ["<u8", "<u4", "<u4", "<u4", "<u8", "<u8", "<u8", "<f4"],
    "offsets": [0, 8, 12, 16, 24, 32, 40, 48],
    "itemsize": 56,
})
APPEND_JOB = np.dtype({
    "names": ["src_key", "src_value", "src_layer_stride", "src_token_stride", "layer_begin", "layer_count",
              "token_count", "dst_slot", "cow_slot", "dst_token", "cow_tokens", "dst_kind", "cow_kind"],
    "formats": ["<u8", "<u8", "<u8", "<u4", "<u4", "<u4", "<u4", "<u4", "<u4", "<u2", "<u2", "u1", "u1"],
    "offsets": [0, 8, 16, 24, 28, 32, 36, 40, 44, 48, 50, 52, 53],
    "itemsize": 56,
})
PREFILL_BLOCK = np.dtype([("item", "<u4"), ("head", "<u2"), ("block", "<u2")])
DESCRIPTOR_PATCH = np.dtype({
    "names": ["table", "first", "count", "source"],
    "formats": ["<u8", "<u4", "<u4", "<u4"],
    "offsets": [0, 8, 12, 16],
    "itemsize": 24,
})

PREFILL_ITEM = np.dtype({
    "names": ["descriptors", "descriptor_count", "token_count", "new_tokens", "layer", "query", "output",
              "attention_scale"],
    "formats": ["<u8", "<u4", "<u4", "<u4", "<u4", "<u8", "<u8", "<f4"],
    "offsets": [0, 8, 12, 16, 20, 24, 32, 40],
    "itemsize": 48,
})
PROMOTION_JOB = np.dtype({
    "names": ["micro_slots", "extent_slot"],
    "formats": [("<u4", (8,)), "<u4"],
    "offsets": [0, 32],
    "itemsize": 36,
})


class KimkvError(RuntimeError):
    def __init__(self, where: str, status: int, native: int = 0):
        super().__init__(f"{where}: {STATUS_NAMES.get(status, status)} (native {native})")
        self.status = status


class Layout(ctypes.Structure):
    _fields_ = [("layers", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32)]


class DecodeLayerArgs(ctypes.Structure):
    """kimkv_decode_layer_args: the layer and each lane's addresses as base + lane * stride (bytes)."""
    _fields_ = [("layer", ctypes.c_uint32), ("attention_scale", ctypes.c_float),
                ("query", ctypes.c_uint64), ("query_stride", ctypes.c_uint64),
                ("output", ctypes.c_uint64), ("output_stride", ctypes.c_uint64),
                ("workspace", ctypes.c_uint64), ("workspace_stride", ctypes.c_uint64),
                ("key", ctypes.c_uint64), ("key_stride", ctypes.c_uint64),
                ("value", ctypes.c_uint64), ("value_stride", ctypes.c_uint64)]


# kimkv_decode_lane (48 bytes): one chunk of a batched decode with its lane's step-constant part.
DECODE_LANE = np.dtype([("descriptors", np.uint64), ("descriptor_count", np.uint32), ("token_count", np.uint32),
                        ("dst_slot", np.uint32), ("cow_slot", np.uint32), ("dst_token", np.uint16),
                        ("cow_tokens", np.uint16), ("dst_kind", np.uint8), ("cow_kind", np.uint8),
                        ("has_write", np.uint8), ("reserved", np.uint8), ("lane", np.uint32),
                        ("first_chunk", np.uint32), ("chunk_count", np.uint32), ("reserved2", np.uint32)])
assert DECODE_LANE.itemsize == 48


class StorageInfo(ctypes.Structure):
    _fields_ = [
        ("layout", Layout), ("micro_capacity", ctypes.c_uint32), ("extent_capacity", ctypes.c_uint32),
        ("micro_page_tokens", ctypes.c_uint16), ("extent_page_tokens", ctypes.c_uint16),
        ("micro_page_elements", ctypes.c_uint64), ("extent_page_elements", ctypes.c_uint64),
        ("micro_reserved_bytes", ctypes.c_uint64), ("extent_reserved_bytes", ctypes.c_uint64),
        ("device", ctypes.c_int), ("compute_units", ctypes.c_int),
    ]


_lib: Optional[ctypes.CDLL] = None

_SIGNATURES = {
    "kimkv_device_count": (ctypes.c_int, []),
    "kimkv_last_native_error": (ctypes.c_int, []),
    "kimkv_device_malloc": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]),
    "kimkv_device_free": (ctypes.c_int, [ctypes.c_void_p]),
    "kimkv_host_malloc_pinned": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]),
    "kimkv_host_free_pinned": (ctypes.c_int, [ctypes.c_void_p]),
    "kimkv_host_malloc_mapped": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p),
                                                ctypes.c_size_t]),
    "kimkv_memcpy_h2d_async": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "kimkv_memcpy_d2h_async": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "kimkv_memcpy_d2d_async": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "kimkv_stream_create": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p)]),
    "kimkv_stream_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "kimkv_stream_synchronize": (ctypes.c_int, [ctypes.c_void_p]),
    "kimkv_device_synchronize": (ctypes.c_int, []),
    "kimkv_event_create": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int]),
    "kimkv_event_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "kimkv_event_record": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "kimkv_stream_wait_event": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "kimkv_event_query": (ctypes.c_int, [ctypes.c_void_p]),
    "kimkv_event_synchronize": (ctypes.c_int, [ctypes.c_void_p]),
    "kimkv_event_elapsed_ms": (ctypes.c_int, [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]),
    "kimkv_storage_create": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), Layout, ctypes.c_uint32,
                                            ctypes.c_uint32, ctypes.c_uint16, ctypes.c_uint16]),
    "kimkv_storage_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "kimkv_storage_query": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(StorageInfo)]),
    "kimkv_storage_page": (ctypes.c_void_p, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32]),
    "kimkv_storage_faults": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32)]),
    "kimkv_append_batch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                          ctypes.c_void_p]),
    "kimkv_gather": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                    ctypes.c_void_p, ctypes.c_void_p]),
    "kimkv_promote_batch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p]),
    "kimkv_patch_descriptors": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]),
    "kimkv_decode_plan": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                         ctypes.POINTER(ctypes.c_uint32), ctypes.c_void_p,
                                         ctypes.POINTER(ctypes.c_uint32)]),
    "kimkv_decode_workspace_bytes": (ctypes.c_size_t, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                                       ctypes.c_uint32]),
    "kimkv_decode_lane_chunks": (ctypes.c_uint32, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]),
    "kimkv_paged_decode_batch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                                ctypes.c_uint32, ctypes.c_void_p]),
    "kimkv_paged_decode_write_batch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                      ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                                      ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]),
    "kimkv_paged_decode_lanes": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                                 ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p,
                                                 ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32,
                                                 ctypes.c_void_p]),
    "kimkv_decode_table_cache_bytes": (ctypes.c_uint64, [ctypes.c_uint32, ctypes.c_uint32]),
    "kimkv_paged_decode_write_batch_slots_prefix": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p,
                                                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32,
                                                                    ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                                                    ctypes.c_void_p, ctypes.c_void_p,
                                                                    ctypes.c_void_p]),
    "kimkv_paged_decode_write_batch_slots": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                            ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                                            ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p,
                                                            ctypes.c_void_p]),
    "kimkv_paged_decode_batch_noalloc": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                        ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                                        ctypes.c_uint32, ctypes.c_void_p]),
    "kimkv_prefill_tokens_per_block": (ctypes.c_uint32, [ctypes.c_void_p, ctypes.c_uint32]),
    "kimkv_paged_prefill_batch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32,
                                                 ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]),
    "kimkv_prefill_order": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                           ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p,
                                           ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32)]),
    "kimkv_paged_prefill_ordered": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32,
                                                   ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                                   ctypes.c_void_p]),
    "kimkv_reference_attention": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                                 ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "kimkv_decode_timing": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                           ctypes.POINTER(ctypes.c_uint64)]),
    "kimkv_prefill_timing": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                            ctypes.POINTER(ctypes.c_uint64)]),
    "kimkv_append_timing": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                           ctypes.POINTER(ctypes.c_uint64)]),
    "kimkv_decode_timing_busy": (ctypes.c_int, [ctypes.POINTER(ctypes.c_double)]),
    "kimkv_linear": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p,
                                    ctypes.c_uint32, ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_void_p]),
    "kimkv_linear_tune": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p,
                                         ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_int,
                                         ctypes.c_float, ctypes.c_void_p]),
    "kimkv_synth_value": (ctypes.c_uint16, [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32]),
    "kimkv_synth_kv_row": (ctypes.c_uint64, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]),
    "kimkv_fill_rows": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                                       ctypes.c_uint32, ctypes.c_void_p]),
    "kimkv_fill_kv": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                     ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]),
    "kimkv_fill_table": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                        ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_void_p]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def lib() -> ctypes.CDLL:
    """Load libkimkv_hip.so (raises when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(status: int, where: str) -> None:
    if status != OK:
        raise KimkvError(where, status, lib().kimkv_last_native_error())


def device_count() -> int:
    return lib().kimkv_device_count()


class DeviceBuffer:
    """Owning device allocation."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        ptr = ctypes.c_void_p()
        check(lib().kimkv_device_malloc(ctypes.byref(ptr), self.nbytes), "device_malloc")
        self.ptr = ptr.value or 0

    def free(self) -> None:
        if self.ptr:
            lib().kimkv_device_free(ctypes.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        handle = ctypes.c_void_p()
        check(lib().kimkv_stream_create(ctypes.byref(handle)), "stream_create")
        self.handle = handle.value

    def synchronize(self) -> None:
        check(lib().kimkv_stream_synchronize(ctypes.c_void_p(self.handle)), "stream_synchronize")

    def destroy(self) -> None:
        if self.handle:
            lib().kimkv_stream_destroy(ctypes.c_void_p(self.handle))
            self.handle = None


class Event:
    def __init__(self, timing: bool = True):
        handle = ctypes.c_void_p()
        check(lib().kimkv_event_create(ctypes.byref(handle), 1 if timing else 0), "event_create")
        self.handle = handle.value

    def record(self, stream: Optional[Stream]) -> None:
        check(lib().kimkv_event_record(ctypes.c_void_p(self.handle), _sh(stream)), "event_record")

    def synchronize(self) -> None:
        check(lib().kimkv_event_synchronize(ctypes.c_void_p(self.handle)), "event_synchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().kimkv_event_elapsed_ms(ctypes.byref(ms), ctypes.c_void_p(self.handle),
                                           ctypes.c_void_p(end.handle)), "event_elapsed")
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                lib().kimkv_event_destroy(ctypes.c_void_p(self.handle))
        except Exception:
            pass


def _sh(stream: Optional[Stream]):
    return ctypes.c_void_p(stream.handle if stream is not None else None)


def upload(array: np.ndarray, stream: Optional[Stream] = None) -> DeviceBuffer:
    array = np.ascontiguousarray(array)
    buf = DeviceBuffer(max(array.nbytes, 1))
    if array.nbytes:
        check(lib().kimkv_memcpy_h2d_async(ctypes.c_void_p(buf.ptr), array.ctypes.data_as(ctypes.c_void_p),
                                           array.nbytes, _sh(stream)), "h2d")
        sync(stream)
    return buf


def copy_to_device(dst_ptr: int, array: np.ndarray, stream: Optional[Stream] = None) -> None:
    array = np.ascontiguousarray(array)
    check(lib().kimkv_memcpy_h2d_async(ctypes.c_void_p(dst_ptr), array.ctypes.data_as(ctypes.c_void_p),
                                       array.nbytes, _sh(stream)), "h2d")
    sync(stream)


def patch_descriptors(patches: np.ndarray, descriptors: np.ndarray, stream: Optional[Stream] = None) -> None:
    """kimkv_patch_descriptors with both arrays uploaded to device memory (waited for)."""
    patches = np.ascontiguousarray(patches, dtype=DESCRIPTOR_PATCH)
    descriptors = np.ascontiguousarray(descriptors, dtype=BLOCK_DESC)
    p, d = upload(patches, stream), upload(descriptors, stream)
    check(lib().kimkv_patch_descriptors(ctypes.c_void_p(p.ptr), len(patches), ctypes.c_void_p(d.ptr), _sh(stream)),
          "patch_descriptors")
    sync(stream)


def download(src_ptr: int, shape, dtype, stream: Optional[Stream] = None) -> np.ndarray:
    out = np.empty(shape, dtype=dtype)
    if out.nbytes:
        check(lib().kimkv_memcpy_d2h_async(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(src_ptr),
                                           out.nbytes, _sh(stream)), "d2h")
        sync(stream)
    return out


def sync(stream: Optional[Stream] = None) -> None:
    if stream is None:
        check(lib().kimkv_device_synchronize(), "device_synchronize")
    else:
        stream.synchronize()


def synth_value(seed: int, row: int, col: int) -> int:
    return int(lib().kimkv_synth_value(seed, row, col))


def synth_kv_row(stream_id: int, layer: int, component: int, token: int) -> int:
    return int(lib().kimkv_synth_kv_row(stream_id, layer, component, token))


def fill_rows(ptr: int, count: int, seed: int, row0: int, cols: int, stream: Optional[Stream] = None) -> None:
    check(lib().kimkv_fill_rows(ctypes.c_void_p(ptr), count, seed, row0, cols, _sh(stream)), "fill_rows")


def fill_kv(ptr: int, layers: int, tokens: int, cols: int, seed: int, stream_id: int, token0: int,
            stream: Optional[Stream] = None) -> None:
    """Synthetic [layers][2][tokens][cols] K/V block (rows synth_kv_row(stream_id, l, c, token0 + t))."""
    check(lib().kimkv_fill_kv(ctypes.c_void_p(ptr), layers, tokens, cols, seed, stream_id, token0, _sh(stream)),
          "fill_kv")


class Storage:
    """Device page pools (kimkv_storage)."""

    def __init__(self, layers: int, kv_heads: int, head_dim: int, micro_capacity: int, extent_capacity: int,
                 micro_tokens: int = 8, extent_tokens: int = 64):
        handle = ctypes.c_void_p()
        check(lib().kimkv_storage_create(ctypes.byref(handle), Layout(layers, kv_heads, head_dim),
                                         micro_capacity, extent_capacity, micro_tokens, extent_tokens),
              "storage_create")
        self.handle = handle.value
        self.layers, self.kv_heads, self.head_dim = layers, kv_heads, head_dim
        self.micro_tokens, self.extent_tokens = micro_tokens, extent_tokens

    @property
    def h(self):
        return ctypes.c_void_p(self.handle)

    def info(self) -> StorageInfo:
        info = StorageInfo()
        check(lib().kimkv_storage_query(self.h, ctypes.byref(info)), "storage_query")
        return info

    def page(self, kind: int, slot: int) -> int:
        return lib().kimkv_storage_page(self.h, kind, slot) or 0

    def faults(self, stream: Optional[Stream] = None) -> tuple[int, int]:
        """kimkv_storage_faults: (status, FAULT_* bits) after waiting for `stream`; clears the word."""
        bits = ctypes.c_uint32()
        status = lib().kimkv_storage_faults(self.h, _sh(stream), ctypes.byref(bits))
        return int(status), int(bits.value)

    def append_batch(self, jobs: np.ndarray, stream: Optional[Stream] = None) -> None:
        jobs = np.ascontiguousarray(jobs, dtype=APPEND_JOB)
        if len(jobs) == 0:
            return
        dev = upload(jobs, stream)
        check(lib().kimkv_append_batch(self.h, ctypes.c_void_p(dev.ptr), len(jobs),
                                       int(jobs["layer_count"].max()), _sh(stream)), "append_batch")
        sync(stream)

    def gather(self, descs: np.ndarray, total_tokens: int, stream: Optional[Stream] = None) -> np.ndarray:
        descs = np.ascontiguousarray(descs, dtype=BLOCK_DESC)
        d = upload(descs, stream)
        n = self.layers * 2 * total_tokens * self.kv_heads * self.head_dim
        out = DeviceBuffer(n * 2)
        check(lib().kimkv_gather(self.h, ctypes.c_void_p(d.ptr), len(descs), total_tokens,
                                 ctypes.c_void_p(out.ptr), _sh(stream)), "gather")
        return download(out.ptr, (n,), np.uint16, stream)

    def promote_batch(self, jobs: np.ndarray, stream: Optional[Stream] = None) -> None:
        jobs = np.ascontiguousarray(jobs, dtype=PROMOTION_JOB)
        if len(jobs) == 0:
            return
        dev = upload(jobs, stream)
        check(lib().kimkv_promote_batch(self.h, ctypes.c_void_p(dev.ptr), len(jobs), _sh(stream)), "promote")
        sync(stream)

    def fill_table(self, descs_ptr: int, count: int, token_begin: int, token_end: int, seed: int,
                   stream_id: int, stream: Optional[Stream] = None) -> None:
        check(lib().kimkv_fill_table(self.h, ctypes.c_void_p(descs_ptr), count, token_begin, token_end, seed,
                                     stream_id, _sh(stream)), "fill_table")

    def decode_plan(self, token_counts, query_heads: int):
        return decode_plan(self.handle, token_counts, query_heads)

    def decode_launch(self, items_ptr: int, prefix_ptr: int, lanes: int, total_chunks: int, chunk_tokens: int,
                      query_heads: int, stream: Optional[Stream] = None) -> None:
        check(lib().kimkv_paged_decode_batch(self.h, ctypes.c_void_p(items_ptr), ctypes.c_void_p(prefix_ptr),
                                             lanes, total_chunks, chunk_tokens, query_heads, _sh(stream)),
              "paged_decode_batch")

    def decode_write_launch(self, items_ptr: int, prefix_ptr: int, lanes: int, total_chunks: int,
                            chunk_tokens: int, query_heads: int, writes_ptr: int,
                            stream: Optional[Stream] = None) -> None:
        """kimkv_paged_decode_write_batch: the decode with each lane's new token (writes[i]) written first."""
        check(lib().kimkv_paged_decode_write_batch(self.h, ctypes.c_void_p(items_ptr), ctypes.c_void_p(prefix_ptr),
                                                   lanes, total_chunks, chunk_tokens, query_heads,
                                                   ctypes.c_void_p(writes_ptr), _sh(stream)),
              "paged_decode_write_batch")

    def decode_write_slots_launch(self, items_ptr: int, prefix_ptr: int, lanes: int, total_chunks: int,
                                  chunk_tokens: int, query_heads: int, writes_ptr: int, slots_ptr: int,
                                  stream: Optional[Stream] = None) -> None:
        """kimkv_paged_decode_write_batch_slots: as decode_write_launch, the merge reading per-lane records
        the decode launch leaves in slots_ptr (lanes x DECODE_LANE_SLOT_BYTES of device memory)."""
        check(lib().kimkv_paged_decode_write_batch_slots(self.h, ctypes.c_void_p(items_ptr),
                                                         ctypes.c_void_p(prefix_ptr), lanes, total_chunks,
                                                         chunk_tokens, query_heads, ctypes.c_void_p(writes_ptr),
                                                         ctypes.c_void_p(slots_ptr), _sh(stream)),
              "paged_decode_write_batch_slots")

    def decode_lanes_launch(self, chunks_ptr: int, lanes: int, total_chunks: int, chunk_tokens: int,
                            query_heads: int, args: DecodeLayerArgs, slots_ptr: int, stream: Optional[Stream] = None,
                            cache_ptr: int = 0, cache_bytes: int = 0, tag: int = 0,
                            host_prefix: Optional[np.ndarray] = None) -> int:
        """kimkv_paged_decode_lanes (chunks_ptr: one DECODE_LANE record per chunk in device memory; args: the
        layer's evenly spaced addresses; cache_ptr/cache_bytes/tag: the optional chunk table cache;
        host_prefix: the optional chunk prefix the merge takes from its arguments instead of slots); returns
        the status."""
        hp = None if host_prefix is None else np.ascontiguousarray(host_prefix, dtype=np.uint32)
        return lib().kimkv_paged_decode_lanes(
            self.h, ctypes.c_void_p(chunks_ptr), lanes, total_chunks, chunk_tokens, query_heads, ctypes.byref(args),
            None if hp is None else hp.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(slots_ptr),
            ctypes.c_void_p(cache_ptr), cache_bytes, tag, _sh(stream))

    def decode_write_slots_prefix_launch(self, items_ptr: int, prefix_ptr: int, host_prefix: np.ndarray,
                                         lanes: int, total_chunks: int, chunk_tokens: int, query_heads: int,
                                         writes_ptr: int, slots_ptr: int, stream: Optional[Stream] = None) -> int:
        """kimkv_paged_decode_write_batch_slots_prefix (host_prefix: the chunk prefix as a host uint32 array,
        carried in the launch's arguments for small launches); returns the status."""
        hp = np.ascontiguousarray(host_prefix, dtype=np.uint32)
        return lib().kimkv_paged_decode_write_batch_slots_prefix(
            self.h, ctypes.c_void_p(items_ptr), ctypes.c_void_p(prefix_ptr), hp.ctypes.data_as(ctypes.c_void_p),
            lanes, total_chunks, chunk_tokens, query_heads, ctypes.c_void_p(writes_ptr), ctypes.c_void_p(slots_ptr),
            _sh(stream))

    def prefill_plan(self, new_token_counts, query_heads: int):
        """(tokens per workgroup, workgroup prefix over items, total workgroups)."""
        per = int(lib().kimkv_prefill_tokens_per_block(self.h, query_heads))
        if per == 0:
            raise KimkvError("prefill_tokens_per_block", 1)
        counts = np.asarray(new_token_counts, dtype=np.uint64)
        prefix = np.zeros(len(counts) + 1, dtype=np.uint32)
        prefix[1:] = np.cumsum((counts + per - 1) // per)
        return per, prefix, int(prefix[-1])

    def prefill_launch(self, items_ptr: int, prefix_ptr: int, item_count: int, total_blocks: int, query_heads: int,
                       stream: Optional[Stream] = None) -> None:
        check(lib().kimkv_paged_prefill_batch(self.h, ctypes.c_void_p(items_ptr), ctypes.c_void_p(prefix_ptr),
                                              item_count, total_blocks, query_heads, _sh(stream)), "paged_prefill_batch")

    def prefill_ordered_launch(self, items_ptr: int, item_count: int, order_ptr: int, order_count: int,
                               query_heads: int, stream: Optional[Stream] = None) -> None:
        check(lib().kimkv_paged_prefill_ordered(self.h, ctypes.c_void_p(items_ptr), item_count,
                                                ctypes.c_void_p(order_ptr), order_count, query_heads, _sh(stream)),
              "paged_prefill_ordered")

    def destroy(self) -> None:
        if self.handle:
            lib().kimkv_storage_destroy(self.h)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


def prefill_order(kv_heads: int, head_dim: int, query_heads: int, compute_units: int, token_counts, new_tokens):
    """kimkv_prefill_order: the workgroup placement of an ordered prefill launch."""
    tc = np.ascontiguousarray(token_counts, dtype=np.uint32)
    nt = np.ascontiguousarray(new_tokens, dtype=np.uint32)
    n = ctypes.c_uint32()
    lib().kimkv_prefill_order(kv_heads, head_dim, query_heads, compute_units, tc.ctypes.data_as(ctypes.c_void_p),
                              nt.ctypes.data_as(ctypes.c_void_p), len(tc), None, 0, ctypes.byref(n))
    order = np.zeros(n.value, dtype=PREFILL_BLOCK)
    check(lib().kimkv_prefill_order(kv_heads, head_dim, query_heads, compute_units,
                                    tc.ctypes.data_as(ctypes.c_void_p), nt.ctypes.data_as(ctypes.c_void_p), len(tc),
                                    order.ctypes.data_as(ctypes.c_void_p), n.value, ctypes.byref(n)),
          "prefill_order")
    return order


DECODE_HEAD_SPLIT = 0x80000000
DECODE_GUIDED = 0x40000000
DECODE_GUIDED_SLICES = 6
DECODE_LANE_SLOT_BYTES = 32
DECODE_ARG_PREFIX_LANES = 64

# Fault bits of kimkv_storage_faults (include/kimkv_hip.h).
FAULT_APPEND_JOB = 0x1
FAULT_DECODE_ITEM = 0x2
FAULT_PREFILL_ITEM = 0x4
FAULT_PROMOTION_JOB = 0x8


def decode_plan(storage_handle: int, token_counts, query_heads: int):
    """kimkv_decode_plan: (chunk_tokens, chunk prefix over lanes, total chunks).  chunk_tokens may carry
    DECODE_HEAD_SPLIT (one kv head per workgroup) or DECODE_GUIDED (persistent slices); pass it to the
    launch, workspace_bytes and lane_chunks unchanged."""
    counts = np.ascontiguousarray(np.asarray(token_counts, dtype=np.uint32))
    prefix = np.zeros(len(counts) + 1, dtype=np.uint32)
    chunk = ctypes.c_uint32()
    total = ctypes.c_uint32()
    check(lib().kimkv_decode_plan(ctypes.c_void_p(storage_handle), counts.ctypes.data_as(ctypes.c_void_p),
                                  len(counts), query_heads, ctypes.byref(chunk),
                                  prefix.ctypes.data_as(ctypes.c_void_p), ctypes.byref(total)), "decode_plan")
    return int(chunk.value), prefix, int(total.value)


def table_cache_bytes(total_chunks: int, chunk_tokens: int) -> int:
    """kimkv_decode_table_cache_bytes: the chunk table cache of a lane-record decode launch."""
    return int(lib().kimkv_decode_table_cache_bytes(total_chunks, chunk_tokens))


def workspace_bytes(token_count: int, chunk_tokens: int, query_heads: int, head_dim: int) -> int:
    return int(lib().kimkv_decode_workspace_bytes(token_count, chunk_tokens, query_heads, head_dim))


def lane_chunks(token_count: int, chunk_tokens: int, head_dim: int) -> int:
    """kimkv_decode_lane_chunks: a lane's chunk (partial slot) count under a planned chunk_tokens."""
    return int(lib().kimkv_decode_lane_chunks(token_count, chunk_tokens, head_dim))


def chunk_prefix(token_counts, chunk_tokens: int, head_dim: int) -> np.ndarray:
    """Running chunk counts over lanes for a chunk_tokens value chosen by the caller."""
    prefix = np.zeros(len(token_counts) + 1, dtype=np.uint32)
    prefix[1:] = np.cumsum([lane_chunks(int(t), chunk_tokens, head_dim) for t in token_counts])
    return prefix


def decode_mode(chunk_tokens: int) -> str:
    """'guided', 'head_split' or 'chunked' for a planned chunk_tokens value."""
    if chunk_tokens & DECODE_GUIDED:
        return "guided"
    return "head_split" if chunk_tokens & DECODE_HEAD_SPLIT else "chunked"


def linear(x_ptr: int, rows: int, in_features: int, w_ptr: int, out_features: int, y_ptr: int, y_f32: bool,
           beta: float, stream: Optional[Stream] = None) -> None:
    """y[rows][out] = x[rows][in] . w[out][in]^T + beta * y (kimkv_linear)."""
    check(lib().kimkv_linear(ctypes.c_void_p(x_ptr), rows, in_features, ctypes.c_void_p(w_ptr), out_features,
                             ctypes.c_void_p(y_ptr), 1 if y_f32 else 0, beta, _sh(stream)), "linear")


def linear_tune(x_ptr: int, rows: int, in_features: int, w_ptrs, out_features: int, y_ptr: int, y_f32: bool,
                beta: float, stream: Optional[Stream] = None) -> None:
    """kimkv_linear_tune: times candidates cycling through the weight
    matrices w_ptrs (y is clobbered)."""
    ws = (ctypes.c_void_p * len(w_ptrs))(*[ctypes.c_void_p(p) for p in w_ptrs])
    check(lib().kimkv_linear_tune(ctypes.c_void_p(x_ptr), rows, in_features, ws, len(w_ptrs), out_features,
                                  ctypes.c_void_p(y_ptr), 1 if y_f32 else 0, beta, _sh(stream)), "linear_tune")


def decode_timing(enable, every: int = 1):
    """Returns (ms, launches) timed since the last call; then times every `every`-th launch if enable."""
    total = ctypes.c_double()
    launches = ctypes.c_uint64()
    check(lib().kimkv_decode_timing(max(1, int(every)) if enable else 0, ctypes.byref(total),
                                    ctypes.byref(launches)), "decode_timing")
    return float(total.value), int(launches.value)


def decode_timing_busy() -> float:
    """Union (ms) of the decode launches timed in the window the last decode_timing call closed."""
    busy = ctypes.c_double()
    check(lib().kimkv_decode_timing_busy(ctypes.byref(busy)), "decode_timing_busy")
    return float(busy.value)


def prefill_timing(enable, every: int = 1):
    """Returns (ms, launches) timed since the last call; then times every `every`-th launch if enable."""
    total = ctypes.c_double()
    launches = ctypes.c_uint64()
    check(lib().kimkv_prefill_timing(max(1, int(every)) if enable else 0, ctypes.byref(total),
                                     ctypes.byref(launches)), "prefill_timing")
    return float(total.value), int(launches.value)


def append_timing(enable, every: int = 1):
    """Returns (ms, launches) of the page-append kernel timed since the last call; then
    times every `every`-th launch if enable."""
    total = ctypes.c_double()
    launches = ctypes.c_uint64()
    check(lib().kimkv_append_timing(max(1, int(every)) if enable else 0, ctypes.byref(total),
                                    ctypes.byref(launches)), "append_timing")
    return float(total.value), int(launches.value)
