"""CPU oracle -- TEST INFRASTRUCTURE ONLY.

ctypes binding of oracle/libkvoracle.so (a plain-C restatement of the
reference's CPU path and kernel data semantics, see kvoracle.h) and of
oracle/_ref/libkimkv_ref.so (the reference's own CPU sources compiled by
oracle/build.py, when they were available at build time).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only to compute expected results or the CPU baseline.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_DIR, "libkvoracle.so")
REF_PATH = os.path.join(_DIR, "_ref", "libkimkv_ref.so")

DESC = np.dtype({
    "names": ["slot", "generation", "logical_token_begin", "valid_tokens", "page_token_capacity", "kind"],
    "formats": ["<u4", "<u4", "<u4", "<u2", "<u2", "u1"],
    "offsets": [0, 4, 8, 12, 14, 16],
    "itemsize": 20,
})


class Layout(ctypes.Structure):
    _fields_ = [("layers", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32)]


class Pools(ctypes.Structure):
    _fields_ = [
        ("layout", Layout), ("micro", ctypes.c_void_p), ("extent", ctypes.c_void_p),
        ("micro_capacity", ctypes.c_uint32), ("extent_capacity", ctypes.c_uint32),
        ("micro_tokens", ctypes.c_uint16), ("extent_tokens", ctypes.c_uint16),
    ]


_lib: Optional[ctypes.CDLL] = None
_ref: Optional[ctypes.CDLL] = None

_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_SIG = {
    "kvo_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
    "kvo_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "kvo_f32_to_f16_array": (None, [_P, _P, ctypes.c_size_t]),
    "kvo_f16_to_f32_array": (None, [_P, _P, ctypes.c_size_t]),
    "kvo_mix64": (ctypes.c_uint64, [ctypes.c_uint64]),
    "kvo_synth": (ctypes.c_uint16, [ctypes.c_uint64, ctypes.c_uint64, _U32]),
    "kvo_kv_row": (ctypes.c_uint64, [_U32, _U32, _U32, _U32]),
    "kvo_synth_rows": (None, [_P, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64, _U32]),
    "kvo_offset": (ctypes.c_size_t, [ctypes.POINTER(Layout), _U32, _U32, _U32, _U32, _U32, _U32]),
    "kvo_page_elements": (ctypes.c_size_t, [ctypes.POINTER(Layout), _U32]),
    "kvo_write_layer_token": (ctypes.c_int, [ctypes.POINTER(Pools), _U32, _U32, _U32, _U32, _P, _P]),
    "kvo_copy_layer_tokens": (ctypes.c_int, [ctypes.POINTER(Pools), _U32, _U32, _U32, _U32, _U32, _U32]),
    "kvo_copy_page_tokens": (ctypes.c_int, [ctypes.POINTER(Pools), _U32, _U32, _U32, _U32, _U32]),
    "kvo_append_tokens": (ctypes.c_int, [ctypes.POINTER(Pools), _P, _U32, _U32, _U32, _U32, _U32, _U32]),
    "kvo_promote": (ctypes.c_int, [ctypes.POINTER(Pools), _P, _U32]),
    "kvo_gather": (ctypes.c_int, [ctypes.POINTER(Pools), _P, _U32, _U32, _P]),
    "kvo_paged_decode": (ctypes.c_int, [ctypes.POINTER(Pools), _P, _U32, _U32, _U32, _U32, _P, ctypes.c_float, _P]),
    "kvo_paged_decode_f32": (ctypes.c_int, [ctypes.POINTER(Pools), _P, _U32, _U32, _U32, _U32, _P, ctypes.c_float,
                                            _P]),
    "kvo_reference_attention": (ctypes.c_int, [ctypes.POINTER(Layout), _P, _U32, _P, _P]),
}


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run __graft_entry__.build()")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIG.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref() -> ctypes.CDLL:
    """The compiled reference CPU library plus the oracle's trace driver."""
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"{REF_PATH} missing (needs /root/reference at build time)")
        _ref = ctypes.CDLL(REF_PATH)
    return _ref


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def f32_to_f16(values) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(values, dtype=np.float32))
    out = np.empty(a.shape, dtype=np.uint16)
    lib().kvo_f32_to_f16_array(_ptr(a), _ptr(out), a.size)
    return out


def f16_to_f32(codes) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(codes, dtype=np.uint16))
    out = np.empty(a.shape, dtype=np.float32)
    lib().kvo_f16_to_f32_array(_ptr(a), _ptr(out), a.size)
    return out


def synth_rows(count: int, seed: int, row0: int, cols: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint16)
    lib().kvo_synth_rows(_ptr(out), count, seed, row0, cols)
    return out


def kv_row(stream: int, layer: int, comp: int, token: int) -> int:
    return int(lib().kvo_kv_row(stream, layer, comp, token))


class HostPools:
    """Host page pools in the reference page layout."""

    def __init__(self, layers, kv_heads, head_dim, micro_capacity, extent_capacity, micro_tokens=8,
                 extent_tokens=64):
        self.layout = Layout(layers, kv_heads, head_dim)
        per_tok = 2 * layers * kv_heads * head_dim
        self.micro = np.zeros(max(1, micro_capacity * micro_tokens * per_tok), dtype=np.uint16)
        self.extent = np.zeros(max(1, extent_capacity * extent_tokens * per_tok), dtype=np.uint16)
        self.pools = Pools(self.layout, self.micro.ctypes.data, self.extent.ctypes.data,
                           micro_capacity, extent_capacity, micro_tokens, extent_tokens)
        self.H, self.D, self.L = kv_heads, head_dim, layers

    def write_layer_token(self, kind, slot, page_token, layer, key, value):
        key = np.ascontiguousarray(key, dtype=np.uint16)
        value = np.ascontiguousarray(value, dtype=np.uint16)
        assert lib().kvo_write_layer_token(ctypes.byref(self.pools), kind, slot, page_token, layer,
                                           _ptr(key), _ptr(value))

    def copy_layer_tokens(self, src_kind, src_slot, dst_kind, dst_slot, count, layer):
        assert lib().kvo_copy_layer_tokens(ctypes.byref(self.pools), src_kind, src_slot, dst_kind, dst_slot,
                                           count, layer)

    def copy_page_tokens(self, src_kind, src_slot, dst_kind, dst_slot, count):
        assert lib().kvo_copy_page_tokens(ctypes.byref(self.pools), src_kind, src_slot, dst_kind, dst_slot, count)

    def append_tokens(self, inp, input_tokens, src_begin, kind, slot, dst_begin, count):
        inp = np.ascontiguousarray(inp, dtype=np.uint16)
        assert lib().kvo_append_tokens(ctypes.byref(self.pools), _ptr(inp), input_tokens, src_begin, kind, slot,
                                       dst_begin, count)

    def promote(self, micro_slots, extent_slot):
        slots = np.ascontiguousarray(np.asarray(micro_slots, dtype=np.uint32))
        assert lib().kvo_promote(ctypes.byref(self.pools), _ptr(slots), extent_slot)

    def gather(self, descs, total_tokens) -> np.ndarray:
        descs = np.ascontiguousarray(descs, dtype=DESC)
        out = np.zeros(self.L * 2 * total_tokens * self.H * self.D, dtype=np.uint16)
        assert lib().kvo_gather(ctypes.byref(self.pools), _ptr(descs), len(descs), total_tokens, _ptr(out))
        return out

    def paged_decode(self, descs, token_count, layer, query_heads, query, scale, f32=False) -> np.ndarray:
        descs = np.ascontiguousarray(descs, dtype=DESC)
        query = np.ascontiguousarray(query, dtype=np.uint16)
        n = query_heads * self.D
        if f32:
            out = np.zeros(n, dtype=np.float32)
            ok = lib().kvo_paged_decode_f32(ctypes.byref(self.pools), _ptr(descs), len(descs), token_count, layer,
                                            query_heads, _ptr(query), scale, _ptr(out))
        else:
            out = np.zeros(n, dtype=np.uint16)
            ok = lib().kvo_paged_decode(ctypes.byref(self.pools), _ptr(descs), len(descs), token_count, layer,
                                        query_heads, _ptr(query), scale, _ptr(out))
        assert ok
        return out


def reference_attention(layers, kv_heads, head_dim, kv, token_count, query) -> np.ndarray:
    layout = Layout(layers, kv_heads, head_dim)
    kv = np.ascontiguousarray(kv, dtype=np.uint16)
    query = np.ascontiguousarray(query, dtype=np.float32)
    out = np.zeros(layers * kv_heads * head_dim, dtype=np.float32)
    ok = lib().kvo_reference_attention(ctypes.byref(layout), _ptr(kv), token_count, _ptr(query), _ptr(out))
    if not ok:
        raise ValueError("reference attention rejected its input")
    return out
