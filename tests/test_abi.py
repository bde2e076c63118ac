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
    assert d.PREFILL_BLOCK.itemsize == 8
    assert d.DECODE_LANE.itemsize == 48      # kimkv_decode_lane (no reference counterpart)
    assert ctypes.sizeof(d.DecodeLayerArgs) == 88


def _block_cost(T, n, b, per=16):
    keys = T - n + min((b + 1) * per, n)
    return (keys + 63) // 64 + 1


def test_prefill_order_places_every_block_once(kimkv):
    """kimkv_prefill_order (host code): every (item, head, block) exactly
    once, idle slots only at the end of an XCD's range, 8 equal ranges, each
    (item, head) pair on one XCD when there are at least 8 pairs, and XCD
    work within one pair's cost of the mean."""
    d = kimkv.device
    rng = np.random.default_rng(5)
    cases = [([1942 + 512, 1430 + 512, 573 + 512, 1103 + 512], [512] * 4),
             ([300, 17, 4000, 900, 65], [280, 17, 33, 900, 64]),
             ([100], [40]), ([], [])]
    cases += [(list(rng.integers(513, 5000, 7)), [512] * 7) for _ in range(3)]
    for totals, news in cases:
        order = d.prefill_order(4, 64, 32, 256, totals, news)
        assert len(order) % 8 == 0
        live = order[order["item"] != 0xFFFFFFFF]
        want = {(i, h, b) for i, n in enumerate(news) for h in range(4) for b in range((n + 15) // 16)}
        got = [(int(e["item"]), int(e["head"]), int(e["block"])) for e in live]
        assert len(got) == len(set(got)) and set(got) == want, (totals, news)
        L = len(order) // 8
        loads, pair_xcd = [], {}
        for x in range(8):
            seg = order[x * L:(x + 1) * L]
            idle = seg["item"] == 0xFFFFFFFF
            assert not np.any(idle[:-1] & ~idle[1:]), "idle slots must trail"
            loads.append(sum(_block_cost(totals[e["item"]], news[e["item"]], e["block"]) for e in seg[~idle]))
            for e in seg[~idle]:
                pair_xcd.setdefault((int(e["item"]), int(e["head"])), set()).add(x)
        if len(pair_xcd) >= 8:
            assert all(len(v) == 1 for v in pair_xcd.values())
            worst_pair = max(sum(_block_cost(totals[i], news[i], b) for b in range((news[i] + 15) // 16))
                             for i in range(len(news)))
            assert max(loads) - min(loads) <= worst_pair
    # Capacity too small: the status says so and the needed size comes back.
    n = ctypes.c_uint32()
    tc = np.array([600], dtype=np.uint32)
    nt = np.array([100], dtype=np.uint32)
    buf = np.zeros(1, dtype=d.PREFILL_BLOCK)
    rc = d.lib().kimkv_prefill_order(4, 64, 32, 256, tc.ctypes.data_as(ctypes.c_void_p),
                                     nt.ctypes.data_as(ctypes.c_void_p), 1, buf.ctypes.data_as(ctypes.c_void_p), 1,
                                     ctypes.byref(n))
    assert rc != 0 and n.value == 32
    assert d.lib().kimkv_prefill_order(4, 64, 30, 256, None, None, 0, None, 0, ctypes.byref(n)) != 0


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
