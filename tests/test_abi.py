"""CPU checks of the C-ABI libraries: they load, export every declared symbol,
the structs have the reference's sizes, and host-side helpers agree with the
oracle.  No GPU call is made."""
import ctypes
import os
import re

import numpy as np

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header: str):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kimkv_[a-z0-9_]+)\s*\(", text)))


def test_device_library_exports_every_declared_symbol(kimkv):
    lib = ctypes.CDLL(kimkv.device.LIB_PATH)
    names = _declared("kimkv_hip.h")
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(kimkv.device.EXPORTED_SYMBOLS) <= set(names)


def test_struct_layouts_match_reference_sizes(kimkv):
    d = kimkv.device
    assert d.BLOCK_DESC.itemsize == 20      # DeviceBlockDescriptor (engine_kv.h:100-127)
    assert d.DECODE_ITEM.itemsize == 56     # DevicePagedDecodeBatchItem (engine_kv.h:172-191)
    assert d.APPEND_JOB.itemsize == 56
    assert d.PROMOTION_JOB.itemsize == 36   # PromotionSlots + target slot
    assert d.PREFILL_ITEM.itemsize == 48


def test_host_synth_matches_oracle(kimkv):
    d = kimkv.device
    rng = np.random.default_rng(0)
    for _ in range(2000):
        seed, row, col = (int(x) for x in rng.integers(0, 2 ** 62, 3))
        col %= 4096
        assert d.synth_value(seed, row, col) == oracle.lib().kvo_synth(seed, row, col)
    assert d.synth_kv_row(3, 21, 1, 32767) == oracle.kv_row(3, 21, 1, 32767)


def test_workspace_never_exceeds_reference_requirement(kimkv):
    d = kimkv.device
    for T in [1, 2, 100, 255, 256, 257, 1000, 4095, 32776]:
        for chunk in [256, 512, 1024, 4096, 8192]:
            ws = d.workspace_bytes(T, chunk, 32, 64)
            assert ws <= 32 * T * 4          # src/cuda/engine/transaction.cpp:56-64
            if T <= chunk:
                assert ws == 0


def test_host_library_exports_every_declared_symbol(kimkv):
    path = os.path.join(os.path.dirname(kimkv.device.LIB_PATH), "libkimkv.so")
    lib = ctypes.CDLL(path)
    names = _declared("kimkv_host.h")
    assert len(names) >= 45
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
