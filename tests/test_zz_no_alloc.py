"""kimkv_paged_decode_batch_noalloc (split-K partials in the library's
file-scope device array) against kimkv_paged_decode_batch (partials in the
lanes' workspaces), both called through the C-ABI: identical output bits on
two calls in a row, the second with a smaller batch, each also within the
decode tolerance of the oracle; a batch whose partials exceed the array is
refused without a launch."""
import ctypes
import math

import numpy as np
import pytest

import oracle
from tests import helpers
from tests.test_gpu_kernels import _input, _populate

pytestmark = pytest.mark.gpu

L, H, D, G = 2, 4, 64, 8
QH = H * G


def _build(dev, token_counts, seed):
    micro_cap = sum(t // 8 + 2 for t in token_counts) + 8
    ext_cap = sum(t // 64 + 1 for t in token_counts) + 2
    storage = dev.Storage(L, H, D, micro_cap, ext_cap)
    pools = oracle.HostPools(L, H, D, micro_cap, ext_cap)
    alloc = helpers.SlotAllocator(micro_cap, ext_cap, seed=seed)
    lanes, keep = [], []
    for i, T in enumerate(token_counts):
        table = helpers.hetero_table(T, alloc)
        keep.append(_populate(dev, storage, pools, table, _input(L, H, D, T, seed=seed * 10 + i)))
        q = oracle.synth_rows(QH * D, seed * 100 + i, 0, D)
        lanes.append((table, T, i % L, q))
    return storage, pools, lanes, keep


def _decode_both(dev, storage, lanes, keep):
    """Runs one planned batch through both entry points; returns (with workspaces, no-alloc) outputs."""
    lib = dev.lib()
    flags, prefix, total = storage.decode_plan([t for (_, t, _, _) in lanes], QH)
    chunk = flags & ~dev.DECODE_HEAD_SPLIT
    assert total > len(lanes), "the case must need split-K partials"
    items_ws = np.zeros(len(lanes), dtype=dev.DECODE_ITEM)
    items_na = np.zeros(len(lanes), dtype=dev.DECODE_ITEM)
    outs_ws, outs_na = [], []
    for i, (table, T, layer, q) in enumerate(lanes):
        dbuf, qbuf = dev.upload(table), dev.upload(q)
        ws = dev.DeviceBuffer(max(dev.workspace_bytes(T, flags, QH, D), 4))
        o1, o2 = dev.DeviceBuffer(QH * D * 2), dev.DeviceBuffer(QH * D * 2)
        items_ws[i] = (dbuf.ptr, len(table), T, layer, qbuf.ptr, ws.ptr, o1.ptr, 1.0 / math.sqrt(D))
        items_na[i] = (dbuf.ptr, len(table), T, layer, qbuf.ptr, 0, o2.ptr, 1.0 / math.sqrt(D))
        keep += [dbuf, qbuf, ws]
        outs_ws.append(o1)
        outs_na.append(o2)
    iw, ina, pb = dev.upload(items_ws), dev.upload(items_na), dev.upload(prefix)
    keep += [iw, ina, pb]
    print(f"no-alloc decode: lanes={len(lanes)} chunk={chunk} chunks={total}", flush=True)
    rc = lib.kimkv_paged_decode_batch(storage.h, ctypes.c_void_p(iw.ptr), ctypes.c_void_p(pb.ptr), len(lanes), total,
                                      flags, QH, None)
    assert rc == dev.OK
    rc = lib.kimkv_paged_decode_batch_noalloc(storage.h, ctypes.c_void_p(ina.ptr), ctypes.c_void_p(pb.ptr),
                                              len(lanes), total, flags, QH, None)
    assert rc == dev.OK
    dev.sync()
    assert storage.faults() == (0, 0)
    get = lambda o: dev.download(o.ptr, (QH * D,), np.uint16)  # noqa: E731
    return [get(o) for o in outs_ws], [get(o) for o in outs_na]


def test_noalloc_decode_matches_workspace_decode(dev):
    # First call: long ragged lanes (several chunks each, split-K merge).
    storage, pools, lanes, keep = _build(dev, [4000, 9000, 300, 12345, 7000], seed=51)
    with_ws, no_alloc = _decode_both(dev, storage, lanes, keep)
    for (table, T, layer, q), a, b in zip(lanes, with_ws, no_alloc):
        assert np.array_equal(a, b), T
        helpers.assert_attention_close(b, pools.paged_decode(table, T, layer, QH, q, 1.0 / math.sqrt(D), f32=True))
    # Second call, smaller batch: the array still holds the first call's partials.
    storage2, pools2, lanes2, keep2 = _build(dev, [2500, 900], seed=52)
    with_ws, no_alloc = _decode_both(dev, storage2, lanes2, keep2)
    for (table, T, layer, q), a, b in zip(lanes2, with_ws, no_alloc):
        assert np.array_equal(a, b), T
        helpers.assert_attention_close(b, pools2.paged_decode(table, T, layer, QH, q, 1.0 / math.sqrt(D), f32=True))


def test_noalloc_decode_refuses_batches_beyond_its_scratch(dev):
    lib = dev.lib()
    storage = dev.Storage(1, H, D, 8, 8)
    per_chunk = QH * (D + 2) * 4
    total = (16 << 20) // per_chunk + 1                # one chunk past the array
    lanes = total // 2
    items = dev.DeviceBuffer(lanes * dev.DECODE_ITEM.itemsize)
    prefix = dev.upload(np.zeros(lanes + 1, dtype=np.uint32))
    dev.copy_to_device(items.ptr, np.zeros(lanes, dtype=dev.DECODE_ITEM))
    rc = lib.kimkv_paged_decode_batch_noalloc(storage.h, ctypes.c_void_p(items.ptr), ctypes.c_void_p(prefix.ptr),
                                              lanes, total, 256, QH, None)
    assert rc == 1                                     # KIMKV_INVALID_ARGUMENT, nothing launched
    dev.sync()
    assert storage.faults() == (0, 0)
