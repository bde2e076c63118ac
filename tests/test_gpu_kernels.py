"""GPU parity of every data-path kernel against the CPU oracle.

Integer/byte work (append, COW, promotion, gather, synthetic fill) must be
bit-exact.  Decode attention must satisfy |gpu - ref| <= 2e-3 + 1e-3*|ref|
against the oracle's fp32-accumulated result on the same seeded inputs.
"""
import math

import numpy as np
import pytest

import oracle
from tests import helpers

pytestmark = pytest.mark.gpu

TINYLLAMA = dict(layers=22, kv_heads=4, head_dim=64)


def _input(L, H, D, T, seed):
    """Contiguous [L][2][T][H][D] synthetic input (fp16 codes)."""
    return oracle.synth_rows(L * 2 * T * H * D, seed, 0, H * D).reshape(L, 2, T, H, D)


def _append_jobs(dev, table, inp_ptr, T, L, H, D):
    jobs = np.zeros(len(table), dtype=dev.APPEND_JOB)
    hd = H * D
    for i, e in enumerate(table):
        b = int(e["logical_token_begin"])
        jobs[i]["src_key"] = inp_ptr + 2 * b * hd
        jobs[i]["src_value"] = inp_ptr + 2 * (T + b) * hd
        jobs[i]["src_layer_stride"] = 2 * T * hd
        jobs[i]["src_token_stride"] = hd
        jobs[i]["layer_begin"] = 0
        jobs[i]["layer_count"] = L
        jobs[i]["token_count"] = int(e["valid_tokens"])
        jobs[i]["dst_slot"] = int(e["slot"])
        jobs[i]["dst_kind"] = int(e["kind"])
        jobs[i]["dst_token"] = 0
    return jobs


def _populate(dev, storage, pools, table, inp):
    L, _, T, H, D = inp.shape
    buf = dev.upload(inp)
    storage.append_batch(_append_jobs(dev, table, buf.ptr, T, L, H, D))
    for e in table:
        pools.append_tokens(inp, T, int(e["logical_token_begin"]), int(e["kind"]), int(e["slot"]), 0,
                            int(e["valid_tokens"]))
    return buf


@pytest.mark.parametrize("shape,T", [((2, 2, 8), 70), ((22, 4, 64), 300), ((3, 1, 12), 9), ((2, 8, 64), 130),
                                     ((2, 2, 64), 200)])
def test_append_gather_bit_exact(dev, shape, T):
    L, H, D = shape
    print(f"append/gather L={L} H={H} D={D} T={T}", flush=True)
    storage = dev.Storage(L, H, D, 64, 8)
    pools = oracle.HostPools(L, H, D, 64, 8)
    table = helpers.hetero_table(T, helpers.SlotAllocator(64, 8, seed=T))
    inp = _input(L, H, D, T, seed=11)
    _populate(dev, storage, pools, table, inp)
    got = storage.gather(table, T)
    assert np.array_equal(got, inp.reshape(-1))
    assert np.array_equal(got, pools.gather(table, T))


def test_patch_descriptors(dev):
    """kimkv_patch_descriptors: whole-table writes (one longer than a
    workgroup's 256 words) and one-entry tail patches land exactly on their
    ranges, all 20 bytes of each entry; entries no patch names keep theirs."""
    rng = np.random.default_rng(11)
    n_tables, cap = 5, 700
    tables = [dev.DeviceBuffer(cap * 20) for _ in range(n_tables)]
    want = []
    for t in tables:
        init = rng.integers(0, 256, (cap, 20), dtype=np.uint8)
        dev.copy_to_device(t.ptr, init)
        want.append(init)
    src = rng.integers(0, 256, (2000, 20), dtype=np.uint8)
    spans = [(0, 0, 600, 0), (1, 3, 1, 600), (2, 699, 1, 601), (3, 10, 52, 602), (4, 0, 1, 654), (4, 1, 645, 655)]
    patches = np.zeros(len(spans), dtype=dev.DESCRIPTOR_PATCH)
    for k, (ti, first, count, source) in enumerate(spans):
        patches[k] = (tables[ti].ptr, first, count, source)
        want[ti][first:first + count] = src[source:source + count]
    dev.patch_descriptors(patches, src.view(dev.BLOCK_DESC).reshape(-1))
    for t, w in zip(tables, want):
        assert np.array_equal(dev.download(t.ptr, (cap, 20), np.uint8), w)
    dev.patch_descriptors(np.zeros(0, dtype=dev.DESCRIPTOR_PATCH), src.view(dev.BLOCK_DESC).reshape(-1))


def test_fill_rows_matches_oracle(dev):
    n = 100003
    buf = dev.DeviceBuffer(n * 2)
    dev.fill_rows(buf.ptr, n, 77, 5, 256)
    got = dev.download(buf.ptr, (n,), np.uint16)
    assert np.array_equal(got, oracle.synth_rows(n, 77, 5, 256))


def test_fill_table_matches_generator(dev):
    L, H, D = 4, 4, 64
    T = 333
    storage = dev.Storage(L, H, D, 64, 8)
    table = helpers.hetero_table(T, helpers.SlotAllocator(64, 8, seed=3))
    d = dev.upload(table)
    storage.fill_table(d.ptr, len(table), 0, T, 99, 5)
    dev.sync()
    got = storage.gather(table, T).reshape(L, 2, T, H * D)
    want = np.empty_like(got)
    for l in range(L):
        for c in range(2):
            for t in range(T):
                want[l, c, t] = oracle.synth_rows(H * D, 99, oracle.kv_row(5, l, c, t), H * D)
    assert np.array_equal(got, want)


def test_single_token_append_with_cow(dev):
    """Engine-style per-layer write into a COW-replaced partial tail
    (src/cuda/engine/transaction.cpp:158-204)."""
    L, H, D = 22, 4, 64
    storage = dev.Storage(L, H, D, 32, 4)
    pools = oracle.HostPools(L, H, D, 32, 4)
    T = 13                                              # pages [0,8) [8,13)
    table = np.array([(3, 1, 0, 8, 8, 0), (9, 1, 8, 5, 8, 0)], dtype=helpers.DESC)
    inp = _input(L, H, D, T, seed=5)
    _populate(dev, storage, pools, table, inp)
    new_kv = oracle.synth_rows(L * 2 * H * D, 123, 0, H * D).reshape(L, 2, H * D)
    buf = dev.upload(new_kv)
    jobs = np.zeros(L, dtype=dev.APPEND_JOB)
    for l in range(L):                                   # one job per layer, COW 5 tokens 9 -> 17
        jobs[l] = (buf.ptr + 2 * (l * 2) * H * D, buf.ptr + 2 * (l * 2 + 1) * H * D, 0, 0, l, 1, 1,
                   17, 9, 5, 5, 0, 0)
    storage.append_batch(jobs)
    for l in range(L):
        pools.copy_layer_tokens(0, 9, 0, 17, 5, l)
        pools.write_layer_token(0, 17, 5, l, new_kv[l, 0], new_kv[l, 1])
    after = np.array([(3, 1, 0, 8, 8, 0), (17, 1, 8, 6, 8, 0)], dtype=helpers.DESC)
    got = storage.gather(after, 14)
    assert np.array_equal(got, pools.gather(after, 14))
    # The shared source tail is untouched.
    assert np.array_equal(storage.gather(table, T), inp.reshape(-1))


def test_promotion_bit_exact(dev):
    L, H, D = 22, 4, 64
    storage = dev.Storage(L, H, D, 32, 4)
    pools = oracle.HostPools(L, H, D, 32, 4)
    T = 70
    slots = [5, 2, 9, 30, 11, 0, 17, 23, 8]
    table = np.array([(slots[i], 1, 8 * i, min(8, T - 8 * i), 8, 0) for i in range(9)], dtype=helpers.DESC)
    inp = _input(L, H, D, T, seed=21)
    _populate(dev, storage, pools, table, inp)
    jobs = np.zeros(1, dtype=dev.PROMOTION_JOB)
    jobs[0]["micro_slots"] = slots[:8]
    jobs[0]["extent_slot"] = 3
    storage.promote_batch(jobs)
    pools.promote(slots[:8], 3)
    promoted = np.array([(3, 1, 0, 64, 64, 1), (slots[8], 1, 64, 6, 8, 0)], dtype=helpers.DESC)
    got = storage.gather(promoted, T)
    assert np.array_equal(got, inp.reshape(-1))
    assert np.array_equal(got, pools.gather(promoted, T))


# ---- decode ---------------------------------------------------------------------

def _run_decode(dev, storage, lanes, query_heads, stream=None, chunk=None):
    """lanes: list of (desc array, token_count, layer, query codes, scale); chunk forces the chunk length."""
    counts = [t for (_, t, _, _, _) in lanes]
    if chunk is None:
        chunk, prefix, total = storage.decode_plan(counts, query_heads)
    else:
        prefix = dev.chunk_prefix(counts, chunk, storage.head_dim)
        total = int(prefix[-1])
    keep = []
    items = np.zeros(len(lanes), dtype=dev.DECODE_ITEM)
    outs = []
    for i, (table, T, layer, q, scale) in enumerate(lanes):
        dbuf = dev.upload(table)
        qbuf = dev.upload(q)
        obuf = dev.DeviceBuffer(query_heads * storage.head_dim * 2)
        wsz = dev.workspace_bytes(T, chunk, query_heads, storage.head_dim)
        wbuf = dev.DeviceBuffer(max(wsz, 4))
        items[i] = (dbuf.ptr, len(table), T, layer, qbuf.ptr, wbuf.ptr if wsz else 0, obuf.ptr, scale)
        keep += [dbuf, qbuf, wbuf]
        outs.append(obuf)
    ibuf = dev.upload(items)
    pbuf = dev.upload(prefix)
    storage.decode_launch(ibuf.ptr, pbuf.ptr, len(lanes), total, chunk, query_heads, stream)
    dev.sync(stream)
    return [dev.download(o.ptr, (query_heads * storage.head_dim,), np.uint16) for o in outs], chunk, total


def _decode_case(dev, shape, token_counts, G, micro_tokens=8, extent_tokens=64, layer=None, seed=1,
                 uniform_pages=None, chunk=None, repeat=1):
    L, H, D = shape
    QH = H * G
    micro_cap = sum(t // micro_tokens + 2 for t in token_counts) + 8
    ext_cap = sum(t // extent_tokens + 1 for t in token_counts) + 2
    storage = dev.Storage(L, H, D, micro_cap, ext_cap, micro_tokens, extent_tokens)
    pools = oracle.HostPools(L, H, D, micro_cap, ext_cap, micro_tokens, extent_tokens)
    alloc = helpers.SlotAllocator(micro_cap, ext_cap, seed=seed, micro_tokens=micro_tokens,
                                  extent_tokens=extent_tokens)
    lanes = []
    keep = []
    for i, T in enumerate(token_counts):
        if uniform_pages:
            table = helpers.uniform_table(T, micro_tokens, alloc)
        else:
            table = helpers.hetero_table(T, alloc)
        inp = _input(L, H, D, T, seed=seed * 100 + i)
        keep.append(_populate(dev, storage, pools, table, inp))
        q = oracle.synth_rows(QH * D, seed * 1000 + i, 0, D)
        lay = (i * 7) % L if layer is None else layer
        lanes.append((table, T, lay, q, 1.0 / math.sqrt(D)))
    wants = [pools.paged_decode(table, T, lay, QH, q, scale, f32=True) for (table, T, lay, q, scale) in lanes]
    worst = 0.0
    first = None
    for _ in range(repeat):
        outs, planned, total = _run_decode(dev, storage, lanes, QH, chunk=chunk)
        for got, want in zip(outs, wants):
            worst = max(worst, helpers.assert_attention_close(got, want))
        if first is None:
            first = outs
        else:   # every launch of the same batch gives the same bits
            assert all(np.array_equal(a, b) for a, b in zip(first, outs))
    chunk = planned
    print(f"decode shape={shape} G={G} T={token_counts} chunk={chunk & 0x3FFFFFFF} mode={dev.decode_mode(chunk)} "
          f"chunks={total} max_err={worst:.2e}", flush=True)
    return chunk, total


def _write_then_decode(dev, fused, tables, T, news, lanes_meta, QH, chunk, shape, seed, cows):
    """One storage populated from `tables`, each lane's new token at position T[i] (into its tail page, a
    fresh page, or a copy-on-write copy of a shared tail), then the decode of T[i] + 1 tokens: by
    kimkv_paged_decode_write_batch (fused) or kimkv_append_batch + kimkv_paged_decode_batch.  Returns the
    outputs and every lane's gathered pages."""
    L, H, D = shape
    micro_cap = sum(t // 8 + 4 for t in T) + 16
    ext_cap = sum(t // 64 + 1 for t in T) + 2
    storage = dev.Storage(L, H, D, micro_cap, ext_cap)
    pools = oracle.HostPools(L, H, D, micro_cap, ext_cap)
    keep = []
    for i, table in enumerate(tables):
        keep.append(_populate(dev, storage, pools, table, _input(L, H, D, T[i], seed=seed * 100 + i)))
    jobs = np.zeros(len(T), dtype=dev.APPEND_JOB)
    ext_tables = []
    src = dev.upload(news)            # [lane][2][H][D]
    for i, table in enumerate(tables):
        layer = lanes_meta[i]
        t = table.copy()
        tail = t[-1]
        j = jobs[i]
        j["src_key"] = src.ptr + 2 * (i * 2) * H * D
        j["src_value"] = src.ptr + 2 * (i * 2 + 1) * H * D
        j["layer_begin"], j["layer_count"], j["token_count"] = layer, 1, 1
        j["dst_kind"] = 0
        if tail["kind"] == 0 and tail["valid_tokens"] < 8 and i in cows:
            # Shared partial tail: continue in a copy (the last free micro slots, distinct per lane).
            new_slot = micro_cap - 1 - i
            j["cow_slot"], j["cow_kind"], j["cow_tokens"] = tail["slot"], 0, tail["valid_tokens"]
            j["dst_slot"], j["dst_token"] = new_slot, tail["valid_tokens"]
            t[-1]["slot"] = new_slot
            t[-1]["valid_tokens"] += 1
        elif tail["kind"] == 0 and tail["valid_tokens"] < 8:
            j["dst_slot"], j["dst_token"] = tail["slot"], tail["valid_tokens"]
            t[-1]["valid_tokens"] += 1
        else:
            new_slot = micro_cap - 1 - i
            j["dst_slot"], j["dst_token"] = new_slot, 0
            # (np.concatenate drops the descriptor's padding: convert back to the 20-byte layout)
            t = np.concatenate([t, np.array([(new_slot, 1, T[i], 1, 8, 0)], dtype=t.dtype)]).astype(helpers.DESC)
        ext_tables.append(t)
    lanes = []
    for i, t in enumerate(ext_tables):
        q = oracle.synth_rows(QH * D, seed * 1000 + i, 0, D)
        lanes.append((t, T[i] + 1, lanes_meta[i], q, 1.0 / math.sqrt(D)))
    counts = [T[i] + 1 for i in range(len(T))]
    prefix = dev.chunk_prefix(counts, chunk, D)
    total = int(prefix[-1])
    items = np.zeros(len(lanes), dtype=dev.DECODE_ITEM)
    outs = []
    for i, (table, n, layer, q, scale) in enumerate(lanes):
        dbuf, qbuf = dev.upload(table), dev.upload(q)
        obuf = dev.DeviceBuffer(QH * D * 2)
        wsz = dev.workspace_bytes(n, chunk, QH, D)
        wbuf = dev.DeviceBuffer(max(wsz, 4))
        items[i] = (dbuf.ptr, len(table), n, layer, qbuf.ptr, wbuf.ptr if wsz else 0, obuf.ptr, scale)
        keep += [dbuf, qbuf, wbuf]
        outs.append(obuf)
    ibuf, pbuf, jbuf = dev.upload(items), dev.upload(prefix), dev.upload(jobs)
    if fused == "slots_prefix":
        # The chunk prefix also in the launch's arguments: a wrong copy is refused without a launch,
        # the right one gives the same pages and outputs.
        slots = dev.DeviceBuffer(len(lanes) * dev.DECODE_LANE_SLOT_BYTES)
        keep.append(slots)
        bad = prefix.copy()
        bad[-1] += 1
        assert storage.decode_write_slots_prefix_launch(ibuf.ptr, pbuf.ptr, bad, len(lanes), total, chunk, QH,
                                                        jbuf.ptr, slots.ptr) == dev.INVALID_ARGUMENT
        assert storage.decode_write_slots_prefix_launch(ibuf.ptr, pbuf.ptr, prefix, len(lanes), total, chunk, QH,
                                                        jbuf.ptr, slots.ptr) == 0
    elif fused == "slots":
        # Merge records in device scratch holding leftovers: random bytes, then a first launch's records
        # (the second launch's tag differs, so none of them may be taken for its own).
        junk = np.random.default_rng(seed).integers(0, 256, len(lanes) * dev.DECODE_LANE_SLOT_BYTES, dtype=np.uint8)
        slots = dev.upload(junk)
        keep.append(slots)
        storage.decode_write_slots_launch(ibuf.ptr, pbuf.ptr, len(lanes), total, chunk, QH, jbuf.ptr, slots.ptr)
        dev.sync()
        for o in outs:
            dev.copy_to_device(o.ptr, np.zeros(QH * D, dtype=np.uint16))
        # The first launch wrote the tokens; the second must not write them again over a copy-on-write
        # source: its jobs write nothing.
        none = jobs.copy()
        none["token_count"] = 0
        jbuf2 = dev.upload(none)
        keep.append(jbuf2)
        storage.decode_write_slots_launch(ibuf.ptr, pbuf.ptr, len(lanes), total, chunk, QH, jbuf2.ptr, slots.ptr)
    elif fused:
        storage.decode_write_launch(ibuf.ptr, pbuf.ptr, len(lanes), total, chunk, QH, jbuf.ptr)
    else:
        storage.append_batch(jobs)
        storage.decode_launch(ibuf.ptr, pbuf.ptr, len(lanes), total, chunk, QH)
    dev.sync()
    assert storage.faults() == (0, 0)
    got = [dev.download(o.ptr, (QH * D,), np.uint16) for o in outs]
    pages = [storage.gather(t, n) for (t, n, _, _, _) in lanes]
    return got, pages, total


@pytest.mark.parametrize("mode", ["four_heads", "head_split", "guided"])
def test_decode_write_batch_matches_append_then_decode(dev, mode):
    """kimkv_paged_decode_write_batch equals kimkv_append_batch of the same jobs followed by
    kimkv_paged_decode_batch, bit for bit in the outputs and the pages: tokens into a partial tail,
    into a fresh page after a full one, and copy-on-write of a shared partial tail; lanes of one chunk and
    of several (the chunk holding the new token writes it)."""
    shape = (3, 4, 64)
    L, H, D = shape
    G = 8
    QH = H * G
    T = [5, 8, 63, 64, 100, 700, 1303, 2049]
    alloc = helpers.SlotAllocator(sum(t // 8 + 4 for t in T) + 16 - len(T) - 4, sum(t // 64 + 1 for t in T) + 2,
                                  seed=21)
    tables = [helpers.hetero_table(t, alloc) for t in T]
    rng = np.random.default_rng(22)
    news = oracle.synth_rows(len(T) * 2 * H * D, 23, 0, D).reshape(len(T), 2, H, D)
    layers = [int(x) for x in rng.integers(0, L, len(T))]
    cows = {0, 4, 6}
    chunk = {"four_heads": 256, "head_split": 256 | dev.DECODE_HEAD_SPLIT, "guided": dev.DECODE_GUIDED | 64}[mode]
    a, pa, total = _write_then_decode(dev, False, tables, T, news, layers, QH, chunk, shape, 24, cows)
    b, pb, _ = _write_then_decode(dev, True, tables, T, news, layers, QH, chunk, shape, 24, cows)
    c, pc, _ = _write_then_decode(dev, "slots", tables, T, news, layers, QH, chunk, shape, 24, cows)
    d, pd, _ = _write_then_decode(dev, "slots_prefix", tables, T, news, layers, QH, chunk, shape, 24, cows)
    assert total > len(T)
    for i in range(len(T)):
        assert np.array_equal(pa[i], pb[i]), (mode, i)
        assert np.array_equal(a[i], b[i]), (mode, i)
        # kimkv_paged_decode_write_batch_slots (and _prefix): the same pages and outputs.
        assert np.array_equal(pa[i], pc[i]), (mode, i)
        assert np.array_equal(a[i], c[i]), (mode, i)
        assert np.array_equal(pa[i], pd[i]), (mode, i)
        assert np.array_equal(a[i], d[i]), (mode, i)
    print(f"decode+write mode={mode} lanes={len(T)} chunks={total}", flush=True)


def test_decode_lane_records_table_cache_head_split_many_rounds(dev):
    """Head-split record launches (one workgroup per chunk and kv head) with a chunk table cache and far
    more workgroups than the GPU holds at once, so the workgroups of a chunk's later heads start after
    its first head's workgroup has stored the table in the same launch.  A launch trusts only tables an
    earlier launch stored: the first launch of a tag and the two after it give the same outputs, bit for
    bit, as the same launch without a cache, and so does a new tag."""
    L, H, D, QH = 1, 4, 64, 32
    n = 40
    T = [4000 + 37 * i for i in range(n)]
    micro_cap, ext_cap = sum(t // 8 + 2 for t in T), sum(t // 64 + 1 for t in T)
    storage = dev.Storage(L, H, D, micro_cap, ext_cap)
    alloc = helpers.SlotAllocator(micro_cap, ext_cap, seed=41)
    chunk = 256 | dev.DECODE_HEAD_SPLIT
    prefix = dev.chunk_prefix(T, chunk, D)
    total = int(prefix[-1])
    assert total * H > 2048                       # several rounds of resident workgroups
    keep = []
    lanes = np.zeros(n, dtype=dev.DECODE_LANE)
    for i, t in enumerate(T):
        table = helpers.hetero_table(t, alloc)
        d = dev.upload(table)
        keep.append(d)
        storage.fill_table(d.ptr, len(table), 0, t, 45, i)
        lanes[i] = (d.ptr, len(table), t, 0, 0, 0, 0, 0, 0, 0, 0, i, prefix[i], prefix[i + 1] - prefix[i], 0)
    chunks = np.concatenate([np.repeat(lanes[i:i + 1], prefix[i + 1] - prefix[i]) for i in range(n)])
    lbuf = dev.upload(chunks)
    qs = dev.upload(np.stack([oracle.synth_rows(QH * D, 4600 + i, 0, D) for i in range(n)]))
    out = dev.upload(np.zeros((n, QH * D), dtype=np.uint16))
    ws_stride = max(max(dev.workspace_bytes(t, chunk, QH, D) for t in T), 256)
    ws = dev.DeviceBuffer(n * ws_stride)
    need = dev.table_cache_bytes(total, chunk)
    cache = dev.upload(np.zeros(need // 2, dtype=np.uint16))
    keep += [lbuf, qs, out, ws, cache]
    a = dev.DecodeLayerArgs()
    a.layer, a.attention_scale = 0, 0.125
    a.query, a.query_stride = qs.ptr, QH * D * 2
    a.output, a.output_stride = out.ptr, QH * D * 2
    a.workspace, a.workspace_stride = ws.ptr, ws_stride
    a.key, a.key_stride = qs.ptr, 0
    a.value, a.value_stride = qs.ptr, 0
    runs = [dict()] + [dict(cache_ptr=cache.ptr, cache_bytes=need, tag=t) for t in (9, 9, 9, 10)]
    zeros = np.zeros((n, QH * D), dtype=np.uint16)
    for kw in runs:
        dev.copy_to_device(out.ptr, zeros)      # every launch writes every output afresh
        assert storage.decode_lanes_launch(lbuf.ptr, n, total, chunk, QH, a, 0, host_prefix=prefix, **kw) == 0
        dev.sync()
        assert storage.faults() == (0, 0)
        got = dev.download(out.ptr, (n, QH * D), np.uint16)
        if not kw:
            first = got
            assert np.any(first != 0)
        else:
            assert np.array_equal(got, first), kw


@pytest.mark.parametrize("mode,order,heads,dim", [("four_heads", 1, 4, 64), ("head_split", 1, 4, 64),
                                                  ("four_heads", -1, 4, 64), ("head_split", -1, 4, 64),
                                                  ("four_heads", 1, 8, 64), ("head_split", 1, 8, 64),
                                                  ("four_heads", 1, 4, 128)])
def test_decode_lane_records_match_item_launch(dev, mode, order, heads, dim):
    """kimkv_paged_decode_lanes (each lane's item and job built in the kernel from a device lane record
    and the layer's evenly spaced addresses) equals kimkv_paged_decode_write_batch_slots_prefix with the
    same items and jobs, bit for bit in the outputs and the pages: tail writes, fresh pages, copy-on-write
    tails, single- and multi-chunk lanes, lanes in address order (order 1) and reversed (order -1: negative
    strides).  With a chunk table cache: the first launch of a tag builds and stores the tables, the next
    two read them, and a new tag over the same cache rebuilds them; every launch gives the same outputs.
    Malformed launches are refused without running.  With 8 kv heads a chunk has two workgroups of four
    heads each (or eight in the head-split mode) sharing its cached table; head_dim 128 takes the generic
    path (and the merge of two dims per lane)."""
    shape = (3, heads, dim)
    L, H, D = shape
    QH, layer = 32, 1
    T = [5, 8, 63, 64, 100, 700, 1303, 2049, 17]
    n = len(T)
    cows = {0, 4, 8}
    alloc = helpers.SlotAllocator(sum(t // 8 + 4 for t in T) + 16 - n - 4, sum(t // 64 + 1 for t in T) + 2, seed=31)
    tables = [helpers.hetero_table(t, alloc) for t in T]
    news = oracle.synth_rows(n * 2 * H * D, 33, 0, D).reshape(n, 2, H, D)
    chunk = {"four_heads": 256, "head_split": 256 | dev.DECODE_HEAD_SPLIT}[mode]
    counts = [t + 1 for t in T]
    prefix = dev.chunk_prefix(counts, chunk, D)
    total = int(prefix[-1])
    assert total > n
    slot_of = list(range(n)) if order == 1 else list(range(n - 1, -1, -1))
    ws_stride = max(max(dev.workspace_bytes(c, chunk, QH, D) for c in counts), 256)

    def run(records):
        micro_cap = sum(t // 8 + 4 for t in T) + 16
        ext_cap = sum(t // 64 + 1 for t in T) + 2
        storage = dev.Storage(L, H, D, micro_cap, ext_cap)
        pools = oracle.HostPools(L, H, D, micro_cap, ext_cap)
        keep = [_populate(dev, storage, pools, table, _input(L, H, D, T[i], seed=3400 + i))
                for i, table in enumerate(tables)]
        # Lane i's rows and buffers sit in slot slot_of[i] of contiguous arrays.
        src = dev.upload(np.stack([news[slot_of.index(k)] for k in range(n)]))
        qs = dev.upload(np.stack([oracle.synth_rows(QH * D, 3500 + slot_of.index(k), 0, D) for k in range(n)]))
        out = dev.upload(np.zeros((n, QH * D), dtype=np.uint16))
        ws = dev.DeviceBuffer(n * ws_stride)
        keep += [src, qs, out, ws]
        jobs = np.zeros(n, dtype=dev.APPEND_JOB)
        items = np.zeros(n, dtype=dev.DECODE_ITEM)
        lanes = np.zeros(n, dtype=dev.DECODE_LANE)
        after = []
        for i, table in enumerate(tables):
            k = slot_of[i]
            t = table.copy()
            tail = t[-1]
            j = jobs[i]
            j["src_key"] = src.ptr + 2 * (k * 2) * H * D
            j["src_value"] = src.ptr + 2 * (k * 2 + 1) * H * D
            j["layer_begin"], j["layer_count"], j["token_count"] = layer, 1, 1
            if tail["kind"] == 0 and tail["valid_tokens"] < 8 and i in cows:
                new_slot = micro_cap - 1 - i
                j["cow_slot"], j["cow_kind"], j["cow_tokens"] = tail["slot"], 0, tail["valid_tokens"]
                j["dst_slot"], j["dst_token"] = new_slot, tail["valid_tokens"]
                t[-1]["slot"] = new_slot
                t[-1]["valid_tokens"] += 1
            elif tail["kind"] == 0 and tail["valid_tokens"] < 8:
                j["dst_slot"], j["dst_token"] = tail["slot"], tail["valid_tokens"]
                t[-1]["valid_tokens"] += 1
            else:
                new_slot = micro_cap - 1 - i
                j["dst_slot"], j["dst_token"] = new_slot, 0
                t = np.concatenate([t, np.array([(new_slot, 1, T[i], 1, 8, 0)], dtype=t.dtype)]).astype(helpers.DESC)
            dbuf = dev.upload(t)
            keep.append(dbuf)
            after.append(t)
            wsz = dev.workspace_bytes(counts[i], chunk, QH, D)
            items[i] = (dbuf.ptr, len(t), counts[i], layer, qs.ptr + k * QH * D * 2,
                        ws.ptr + k * ws_stride if wsz else 0, out.ptr + k * QH * D * 2, 0.125)
            lanes[i] = (dbuf.ptr, len(t), counts[i], j["dst_slot"], j["cow_slot"], j["dst_token"], j["cow_tokens"],
                        j["dst_kind"], j["cow_kind"], 1, 0, i, prefix[i], prefix[i + 1] - prefix[i], 0)
        slots = dev.DeviceBuffer(n * dev.DECODE_LANE_SLOT_BYTES)
        pbuf = dev.upload(prefix)
        keep += [slots, pbuf]
        if records:
            chunks = np.concatenate([np.repeat(lanes[i:i + 1], prefix[i + 1] - prefix[i]) for i in range(n)])
            assert len(chunks) == total
            lbuf = dev.upload(chunks)
            keep.append(lbuf)
            step = -1 if order == -1 else 1
            a = dev.DecodeLayerArgs()
            a.layer, a.attention_scale = layer, 0.125
            m = 1 << 64
            a.query, a.query_stride = qs.ptr + slot_of[0] * QH * D * 2, (step * QH * D * 2) % m
            a.output, a.output_stride = out.ptr + slot_of[0] * QH * D * 2, (step * QH * D * 2) % m
            a.workspace, a.workspace_stride = ws.ptr + slot_of[0] * ws_stride, (step * ws_stride) % m
            a.key, a.key_stride = src.ptr + slot_of[0] * 4 * H * D, (step * 4 * H * D) % m
            a.value, a.value_stride = src.ptr + slot_of[0] * 4 * H * D + 2 * H * D, (step * 4 * H * D) % m
            assert storage.decode_lanes_launch(lbuf.ptr, n, total, chunk, QH, a,
                                               0) == dev.INVALID_ARGUMENT     # split lanes need merge records
            assert storage.decode_lanes_launch(lbuf.ptr, n, total, dev.DECODE_GUIDED | 64, QH, a,
                                               slots.ptr) == dev.INVALID_ARGUMENT
            assert storage.decode_lanes_launch(lbuf.ptr, 69, total, chunk, QH, a,
                                               slots.ptr) == dev.INVALID_ARGUMENT     # more than 64 lanes
            need = dev.table_cache_bytes(total, chunk)
            cache = dev.upload(np.full(need // 2, 0x7777, dtype=np.uint16))    # leftovers, no valid tag
            keep.append(cache)
            assert storage.decode_lanes_launch(lbuf.ptr, n, total, chunk, QH, a, slots.ptr,
                                               cache_ptr=cache.ptr, cache_bytes=need - 16,
                                               tag=5) == dev.INVALID_ARGUMENT       # cache too small
            assert storage.decode_lanes_launch(lbuf.ptr, n, total, chunk, QH, a, slots.ptr,
                                               cache_ptr=cache.ptr, cache_bytes=need,
                                               tag=0) == dev.INVALID_ARGUMENT       # tag 0 is reserved
            # Records that do not describe their chunk (a lane past lane_count, a chunk range that
            # misses the chunk) are reported by the workgroup and skipped.
            wrong = chunks.copy()
            wrong[0]["lane"] = n
            wrong[total - 1]["first_chunk"] = total
            wbuf = dev.upload(wrong)
            keep.append(wbuf)
            assert storage.decode_lanes_launch(wbuf.ptr, n, total, chunk, QH, a, slots.ptr) == 0
            status, bits = storage.faults()
            assert status == dev.INVALID_ARGUMENT and bits & dev.FAULT_DECODE_ITEM, (status, bits)
            bad = prefix.copy()
            bad[-1] += 1
            assert storage.decode_lanes_launch(lbuf.ptr, n, total, chunk, QH, a, 0,
                                               host_prefix=bad) == dev.INVALID_ARGUMENT   # ends past total
            bad = prefix.copy()
            bad[1] = bad[0]
            assert storage.decode_lanes_launch(lbuf.ptr, n, total, chunk, QH, a, 0,
                                               host_prefix=bad) == dev.INVALID_ARGUMENT   # a lane without chunks
            # Merge from slots, then from the prefix in its arguments (no slots), each with and
            # without the table cache: every output the same.
            runs = [dict()] + [dict(cache_ptr=cache.ptr, cache_bytes=need, tag=t) for t in (5, 5, 5, 6)]
            runs += [dict(host_prefix=prefix, slots=0), dict(host_prefix=prefix, slots=0, cache_ptr=cache.ptr,
                                                               cache_bytes=need, tag=7),
                     dict(host_prefix=prefix, slots=0, cache_ptr=cache.ptr, cache_bytes=need, tag=7)]
            for kw in runs:
                kw = dict(kw)
                sp = kw.pop("slots", slots.ptr)
                assert storage.decode_lanes_launch(lbuf.ptr, n, total, chunk, QH, a, sp, **kw) == 0
                dev.sync()
                snap = dev.download(out.ptr, (n, QH * D), np.uint16)
                if kw:
                    assert np.array_equal(snap, first), kw
                else:
                    first = snap
        else:
            ibuf, jbuf = dev.upload(items), dev.upload(jobs)
            keep += [ibuf, jbuf]
            assert storage.decode_write_slots_prefix_launch(ibuf.ptr, pbuf.ptr, prefix, n, total, chunk, QH,
                                                            jbuf.ptr, slots.ptr) == 0
        dev.sync()
        assert storage.faults() == (0, 0)
        got = dev.download(out.ptr, (n, QH * D), np.uint16)
        outs = [got[slot_of[i]] for i in range(n)]
        pages = [storage.gather(t, counts[i]) for i, t in enumerate(after)]
        return outs, pages

    a_out, a_pages = run(False)
    b_out, b_pages = run(True)
    for i in range(n):
        assert np.array_equal(a_pages[i], b_pages[i]), (mode, order, i)
        assert np.array_equal(a_out[i], b_out[i]), (mode, order, i)
    print(f"lane records mode={mode} order={order} lanes={n} chunks={total}", flush=True)


def _fused_case(dev, shape, lanes, chunk, micro_tokens=8, extent_tokens=64, seed=70, QH=None):
    """Write-and-decode launches against the oracle and against append-then-decode, with explicit jobs.

    lanes: (table before, mode, layer) with mode "tail" (the new token goes into the tail page),
    "cow" (the tail's valid tokens are copied into a fresh page of the tail's kind, the new token
    after them), ("cow_short", n) (only the first n tokens copied, the new token still after the
    tail's valid count) or "fresh" (a new micro page).  Pages must match the oracle's bit for bit and
    outputs the oracle within tolerance; outputs must also equal append-then-decode bit for bit,
    except for "cow_short" lanes, whose fused chunk holding the destination page takes the generic
    path (kept and copied positions share an 8-token group) while append-then-decode reads the
    written page on the fast path.  Returns the worst error against the oracle."""
    L, H, D = shape
    QH = QH or 8 * H
    cap = {helpers.MICRO: micro_tokens, helpers.EXTENT: extent_tokens}
    used = {helpers.MICRO: set(), helpers.EXTENT: set()}
    for table, _, _ in lanes:
        for e in table:
            used[int(e["kind"])].add(int(e["slot"]))
    micro_cap = max(used[helpers.MICRO] | {0}) + len(lanes) + 4
    ext_cap = max(used[helpers.EXTENT] | {0}) + len(lanes) + 4
    spare = {helpers.MICRO: [s for s in range(micro_cap) if s not in used[helpers.MICRO]],
             helpers.EXTENT: [s for s in range(ext_cap) if s not in used[helpers.EXTENT]]}
    news = oracle.synth_rows(len(lanes) * 2 * H * D, seed + 1, 0, D).reshape(len(lanes), 2, H, D)
    plans = []
    for i, (table, mode, layer) in enumerate(lanes):
        T = int(table[-1]["logical_token_begin"]) + int(table[-1]["valid_tokens"])
        tail = table[-1]
        kind, valid = int(tail["kind"]), int(tail["valid_tokens"])
        after = table.copy()
        job = dict(dst_kind=helpers.MICRO, dst_slot=0, dst_token=0, cow_kind=0, cow_slot=0, cow_tokens=0)
        if mode == "tail":
            assert valid < cap[kind]
            job.update(dst_kind=kind, dst_slot=int(tail["slot"]), dst_token=valid)
            after[-1]["valid_tokens"] += 1
        elif mode == "fresh":
            slot = spare[helpers.MICRO].pop()
            job.update(dst_kind=helpers.MICRO, dst_slot=slot)
            after = np.concatenate([after, np.array([(slot, 1, T, 1, micro_tokens, helpers.MICRO)],
                                                    dtype=after.dtype)]).astype(helpers.DESC)
        else:
            assert valid < cap[kind]
            n = valid if mode == "cow" else mode[1]
            slot = spare[kind].pop()
            job.update(dst_kind=kind, dst_slot=slot, dst_token=valid, cow_kind=kind, cow_slot=int(tail["slot"]),
                       cow_tokens=n)
            after[-1]["slot"] = slot
            after[-1]["valid_tokens"] += 1
        plans.append((table, after, T, layer, job))

    def run(fused):
        storage = dev.Storage(L, H, D, micro_cap, ext_cap, micro_tokens, extent_tokens)
        pools = oracle.HostPools(L, H, D, micro_cap, ext_cap, micro_tokens, extent_tokens)
        keep = []
        for i, (table, _, T, _, _) in enumerate(plans):
            keep.append(_populate(dev, storage, pools, table, _input(L, H, D, T, seed=seed * 100 + i)))
        src = dev.upload(news)
        jobs = np.zeros(len(plans), dtype=dev.APPEND_JOB)
        for i, (_, _, _, layer, job) in enumerate(plans):
            j = jobs[i]
            j["src_key"] = src.ptr + 2 * (i * 2) * H * D
            j["src_value"] = src.ptr + 2 * (i * 2 + 1) * H * D
            j["layer_begin"], j["layer_count"], j["token_count"] = layer, 1, 1
            for k, v in job.items():
                j[k] = v
            if job["cow_tokens"]:
                pools.copy_layer_tokens(job["cow_kind"], job["cow_slot"], job["dst_kind"], job["dst_slot"],
                                        job["cow_tokens"], layer)
            pools.write_layer_token(job["dst_kind"], job["dst_slot"], job["dst_token"], layer, news[i, 0], news[i, 1])
        counts = [T + 1 for (_, _, T, _, _) in plans]
        prefix = dev.chunk_prefix(counts, chunk, D)
        total = int(prefix[-1])
        items = np.zeros(len(plans), dtype=dev.DECODE_ITEM)
        outs, wants = [], []
        for i, (_, after, T, layer, _) in enumerate(plans):
            q = oracle.synth_rows(QH * D, seed * 1000 + i, 0, D)
            dbuf, qbuf = dev.upload(after), dev.upload(q)
            obuf = dev.DeviceBuffer(QH * D * 2)
            wsz = dev.workspace_bytes(T + 1, chunk, QH, D)
            wbuf = dev.DeviceBuffer(max(wsz, 4))
            items[i] = (dbuf.ptr, len(after), T + 1, layer, qbuf.ptr, wbuf.ptr if wsz else 0, obuf.ptr, 0.125)
            keep += [dbuf, qbuf, wbuf]
            outs.append(obuf)
            wants.append(pools.paged_decode(after, T + 1, layer, QH, q, 0.125, f32=True))
        ibuf, pbuf, jbuf = dev.upload(items), dev.upload(prefix), dev.upload(jobs)
        if fused:
            storage.decode_write_launch(ibuf.ptr, pbuf.ptr, len(plans), total, chunk, QH, jbuf.ptr)
        else:
            storage.append_batch(jobs)
            storage.decode_launch(ibuf.ptr, pbuf.ptr, len(plans), total, chunk, QH)
        dev.sync()
        assert storage.faults() == (0, 0)
        got = [dev.download(o.ptr, (QH * D,), np.uint16) for o in outs]
        pages = [storage.gather(after, T + 1) for (_, after, T, _, _) in plans]
        want_pages = [pools.gather(after, T + 1) for (_, after, T, _, _) in plans]
        return got, pages, wants, want_pages, total

    a, pa, wants, want_pages, total = run(False)
    b, pb, _, _, _ = run(True)
    worst = 0.0
    for i, (_, mode, _) in enumerate(lanes):
        assert np.array_equal(pb[i], want_pages[i]), i
        assert np.array_equal(pa[i], pb[i]), i
        helpers.assert_attention_close(a[i], wants[i])
        if not isinstance(mode, tuple):
            assert np.array_equal(a[i], b[i]), i
        worst = max(worst, helpers.assert_attention_close(b[i], wants[i]))
    print(f"fused write+decode chunk={chunk & 0x3FFFFFFF} mode={dev.decode_mode(chunk)} chunks={total} "
          f"pages={micro_tokens}/{extent_tokens} max_err={worst:.2e}", flush=True)
    return worst


@pytest.mark.parametrize("mode", ["four_heads", "head_split", "guided"])
def test_decode_write_batch_unaligned_pages_cow_across_chunks(dev, mode):
    """6-token micro / 48-token extent pages (not 8-aligned: the generic path): copy-on-write tails
    that start in one chunk and end in the next (tokens [252, 258) with 256-token chunks), so the
    earlier chunk's workgroup reads copied positions while the later one stores them.  Every chunk
    takes copied positions from the source page and the new token from the job's rows, so the
    fused launch equals append-then-decode bit for bit and the oracle within tolerance."""
    shape = (2, 4, 64)
    alloc = helpers.SlotAllocator(400, 8, seed=71, micro_tokens=6, extent_tokens=48)
    lanes = [(helpers.uniform_table(257, 6, alloc), "cow", 1),      # tail [252, 257): crosses 256
             (helpers.uniform_table(250, 6, alloc), "cow", 0),
             (helpers.uniform_table(253, 6, alloc), "tail", 1),
             (helpers.uniform_table(511, 6, alloc), "tail", 0),     # tail [510, 511)
             (helpers.uniform_table(300, 6, alloc), "fresh", 1),
             (helpers.uniform_table(515, 6, alloc), ("cow_short", 2), 0)]
    chunk = {"four_heads": 256, "head_split": 256 | dev.DECODE_HEAD_SPLIT, "guided": dev.DECODE_GUIDED | 64}[mode]
    _fused_case(dev, shape, lanes, chunk, micro_tokens=6, extent_tokens=48)


@pytest.mark.parametrize("mode", ["four_heads", "head_split"])
def test_decode_write_batch_fast_path_redirects(dev, mode):
    """8/64-token pages (fast path): an extent tail at token 8 (not 64-aligned) copied on write across
    a chunk boundary (chunk 0 reads copied positions of the destination from the source page), a
    micro copy-on-write tail, copies shorter than the tail (generic path), a new token that lands on
    a full 64-token step, and plain tail writes; fused equals append-then-decode bit for bit."""
    shape = (3, 4, 64)
    alloc = helpers.SlotAllocator(200, 64, seed=72)

    def ext_at_8(valid):
        return np.array([(alloc.take(helpers.MICRO), 1, 0, 8, 8, helpers.MICRO),
                         (alloc.take(helpers.EXTENT), 1, 8, valid, 64, helpers.EXTENT)], dtype=helpers.DESC)

    lanes = [(ext_at_8(60), "cow", 2),                          # extent [8, 68) -> copy; new token 68
             (ext_at_8(30), "cow", 1),
             (ext_at_8(55), "tail", 0),
             (helpers.hetero_table(127, alloc), "tail", 1),     # new token 127: last of a full step
             (helpers.hetero_table(1003, alloc), "cow", 2),         # micro tail [1000, 1003)
             (helpers.hetero_table(1005, alloc), ("cow_short", 1), 0),
             (helpers.hetero_table(512, alloc), "fresh", 1),
             (helpers.hetero_table(64 * 5 + 6, alloc), "cow", 0)]
    chunk = {"four_heads": 64, "head_split": 64 | dev.DECODE_HEAD_SPLIT}[mode]
    _fused_case(dev, shape, lanes, chunk)
    _fused_case(dev, shape, lanes, chunk + 192)


def test_decode_zero_token_lane_beside_split_lane(dev):
    """A lane of no tokens gets one (skipped) chunk from the planner, so a batch of lanes [0, 300]
    still runs the split-K merge for the 300-token lane, through kimkv_paged_decode_batch and the
    no-alloc entry point; the empty lane's output is left untouched.  A prefix that gives the empty
    lane no chunk ([0, 0, 2]: as many chunks as lanes) would skip the merge: the split lane is then
    reported and skipped instead of left unmerged, and nothing is written past the chunks."""
    import ctypes
    L, H, D, G = 1, 4, 64, 8
    QH = H * G
    storage = dev.Storage(L, H, D, 64, 16)
    pools = oracle.HostPools(L, H, D, 64, 16)
    alloc = helpers.SlotAllocator(64, 16, seed=73)
    table = helpers.hetero_table(300, alloc)
    keep = [_populate(dev, storage, pools, table, _input(L, H, D, 300, seed=74))]
    q = oracle.synth_rows(QH * D, 75, 0, D)
    want = pools.paged_decode(table, 300, 0, QH, q, 0.125, f32=True)
    chunk = 256
    prefix = dev.chunk_prefix([0, 300], chunk, D)
    assert list(prefix) == [0, 1, 3]
    flags, planned, total = storage.decode_plan([0, 300], QH)
    assert planned[1] == 1 and total == planned[2]   # the zero-token lane has one chunk
    dbuf, qbuf = dev.upload(table), dev.upload(q)
    sentinel = np.full(QH * D, 0x7E00, dtype=np.uint16)
    lib = dev.lib()
    for noalloc in (False, True):
        outs = [dev.upload(sentinel), dev.upload(sentinel)]
        ws = dev.DeviceBuffer(dev.workspace_bytes(300, chunk, QH, D))
        items = np.zeros(2, dtype=dev.DECODE_ITEM)
        items[0] = (dbuf.ptr, len(table), 0, 0, qbuf.ptr, 0, outs[0].ptr, 0.125)
        items[1] = (dbuf.ptr, len(table), 300, 0, qbuf.ptr, 0 if noalloc else ws.ptr, outs[1].ptr, 0.125)
        ibuf, pbuf = dev.upload(items), dev.upload(prefix)
        fn = lib.kimkv_paged_decode_batch_noalloc if noalloc else lib.kimkv_paged_decode_batch
        print(f"zero-token lane: noalloc={noalloc} prefix={list(prefix)}", flush=True)
        assert fn(storage.h, ctypes.c_void_p(ibuf.ptr), ctypes.c_void_p(pbuf.ptr), 2, 3, chunk, QH, None) == 0
        dev.sync()
        assert storage.faults() == (0, 0)
        assert np.array_equal(dev.download(outs[0].ptr, (QH * D,), np.uint16), sentinel)
        helpers.assert_attention_close(dev.download(outs[1].ptr, (QH * D,), np.uint16), want)
        # The inconsistent plan: no chunk for the empty lane, two for the other.
        bad = np.array([0, 0, 2], dtype=np.uint32)
        out2 = dev.upload(sentinel)
        items[1]["output"] = out2.ptr
        ibuf2, pbuf2 = dev.upload(items), dev.upload(bad)
        assert fn(storage.h, ctypes.c_void_p(ibuf2.ptr), ctypes.c_void_p(pbuf2.ptr), 2, 2, chunk, QH, None) == 0
        dev.sync()
        assert storage.faults() == (1, dev.FAULT_DECODE_ITEM)
        assert np.array_equal(dev.download(out2.ptr, (QH * D,), np.uint16), sentinel)
        keep += [ws, ibuf, pbuf, ibuf2, pbuf2, out2] + outs
    del keep


def test_decode_guided_streams_own_counter_slots(dev):
    """Guided launches take the work-counter slot of their stream: interleaved launches on several
    streams stay correct, and a storage refuses a guided launch from a 65th distinct stream (no slot
    left) without launching, while streams that own a slot keep working."""
    L, H, D, G = 1, 4, 64, 8
    QH = H * G
    storage = dev.Storage(L, H, D, 256, 64)
    pools = oracle.HostPools(L, H, D, 256, 64)
    alloc = helpers.SlotAllocator(256, 64, seed=76)
    lanes, keep = [], []
    for i, T in enumerate([700, 2000, 90]):
        table = helpers.hetero_table(T, alloc)
        keep.append(_populate(dev, storage, pools, table, _input(L, H, D, T, seed=77 + i)))
        lanes.append((table, T, 0, oracle.synth_rows(QH * D, 80 + i, 0, D), 0.125))
    wants = [pools.paged_decode(t, T, 0, QH, q, s, f32=True) for (t, T, _, q, s) in lanes]
    GU = dev.DECODE_GUIDED | 64
    streams = [dev.Stream() for _ in range(64)]
    for rnd in range(2):
        for k, st in enumerate(streams):
            if rnd == 1 and k % 8 != 0:
                continue
            outs, _, _ = _run_decode(dev, storage, lanes, QH, stream=st, chunk=GU)
            for got, want in zip(outs, wants):
                helpers.assert_attention_close(got, want)
    extra = dev.Stream()
    with pytest.raises(dev.KimkvError):
        _run_decode(dev, storage, lanes, QH, stream=extra, chunk=GU)
    outs, _, _ = _run_decode(dev, storage, lanes, QH, stream=streams[5], chunk=GU)
    for got, want in zip(outs, wants):
        helpers.assert_attention_close(got, want)
    for st in streams + [extra]:
        st.destroy()
    del keep


def test_decode_config1_tinyllama(dev):
    """One TinyLlama layer, 4 lanes at {17,100,513,1000} + 1 appended token."""
    _decode_case(dev, (1, 4, 64), [18, 101, 514, 1001], G=8, layer=0)


def test_decode_single_token_lane_is_value(dev):
    _decode_case(dev, (2, 4, 64), [1, 2, 7, 8, 9, 63, 64, 65], G=8)


def test_decode_split_k_long_lanes(dev):
    chunk, total = _decode_case(dev, (22, 4, 64), [4000, 9000, 300, 12345], G=8, seed=4)
    assert total > 4          # several lanes split across chunks -> combine path


def test_decode_combine_wide_heads_and_many_chunks(dev):
    # Split-K merges with 2 and 4 dims per lane (D = 128, 256; generic path)
    # and a lane of more than 64 chunks (the merge folds rounds of 64).
    chunk, total = _decode_case(dev, (1, 2, 128), [300, 2600], G=4, seed=13)
    assert total > 2
    chunk, total = _decode_case(dev, (1, 1, 256), [700, 2000], G=2, seed=14)
    assert total > 2
    chunk, total = _decode_case(dev, (1, 4, 64), [20000, 33], G=8, seed=15)
    length = chunk & ~dev.DECODE_HEAD_SPLIT
    assert (20000 + length - 1) // length > 64


def test_decode_full_step_counts(dev):
    # Chunks of 1..9 full 64-token steps, odd and even, with and without a tail.
    _decode_case(dev, (2, 4, 64), [128, 192, 256, 320, 389, 447, 511, 576], G=8, seed=16)
    _decode_case(dev, (1, 4, 64), [4096 + 64 * 3, 4096 + 77, 8192], G=8, seed=17)


def test_decode_plan_balances_long_lanes(dev):
    storage = dev.Storage(1, 4, 64, 16, 16)
    cus = storage.info().compute_units
    H = 4
    for lanes, T in [(256, 32769), (128, 32769), (64, 32769), (256, 32768), (60, 1600), (3, 12345), (1, 1),
                     (4, 200000), (64, 8192), (60, 20000)]:
        flags, prefix, total = storage.decode_plan([T] * lanes, 32)
        assert not flags & dev.DECODE_GUIDED, (lanes, T, flags)   # the guided mode is opt-in
        split = bool(flags & dev.DECODE_HEAD_SPLIT)
        chunk = flags & ~dev.DECODE_HEAD_SPLIT
        n = (T + chunk - 1) // chunk
        assert chunk % 64 == 0 and 256 <= chunk <= 65536
        assert total == lanes * n and list(prefix) == [i * n for i in range(lanes + 1)]
        # The lane's chunks are even: the last one is short by less than 64 tokens per chunk.
        assert n * chunk - T < 64 * n or chunk == 256
        # About one round of resident workgroups (two per CU): four kv heads per workgroup, or
        # one head per workgroup when that spares the split-K merge.
        blocks = total * (H if split else 1)
        if lanes * T * H >= 2 * cus * T and T <= 65536:
            assert split and n == 1, (lanes, T, flags)
        elif lanes * T >= 2 * cus * 256:
            assert not split and blocks <= 2 * cus + lanes, (lanes, T, flags)
    ragged = [100, 5000, 32769, 7]
    flags, prefix, total = storage.decode_plan(ragged, 32)
    chunk = flags & ~dev.DECODE_HEAD_SPLIT
    assert total == sum((t + chunk - 1) // chunk for t in ragged)
    # Guided lanes: min(6, max(1, T / (D + 2))) slices, so a lane's partials
    # never exceed the reference's QH * T float workspace.
    for T in [1, 65, 66, 131, 132, 395, 396, 1000, 32769]:
        n = dev.lane_chunks(T, dev.DECODE_GUIDED | 64, 64)
        assert n == min(6, max(1, T // 66)), (T, n)
        assert dev.workspace_bytes(T, dev.DECODE_GUIDED | 64, 32, 64) <= 32 * T * 4


def test_decode_guided_slices(dev):
    # Persistent workgroups taking (slice, lane, kv head) units from the
    # device counter: ragged lanes with one to six slices (one-slice lanes
    # written directly, empty slices from 64-alignment), the longest slices
    # the table holds (T/2 <= 65536), group sizes 16 and 1, generic head dims
    # and unaligned pages (generic wave path), and many launches in a row
    # (counter slots reused after their reset).
    GU = dev.DECODE_GUIDED | 64
    _decode_case(dev, (2, 4, 64), [1, 5, 66, 100, 131, 396, 397, 4000, 12345, 33000], G=8, seed=60, chunk=GU)
    _decode_case(dev, (1, 4, 64), [130000, 70000, 64, 8193], G=8, seed=61, chunk=GU)
    _decode_case(dev, (2, 2, 64), [700, 9000], G=16, seed=62, chunk=GU)
    _decode_case(dev, (2, 8, 64), [333, 5000], G=1, seed=63, chunk=GU)
    _decode_case(dev, (1, 2, 128), [90, 1500, 3000], G=4, seed=64, chunk=GU)
    _decode_case(dev, (2, 4, 64), [17, 200, 3000], G=8, micro_tokens=6, extent_tokens=48, seed=65,
                 uniform_pages=True, chunk=GU)
    # 70 launches on one storage: its 64 counter slots are reused after their reset.
    _decode_case(dev, (1, 4, 64), [300, 1000, 2500], G=8, seed=66, chunk=GU, repeat=70)


def test_decode_long_chunks(dev):
    # The longest chunks the kernel takes (65536 tokens: an 8192-entry group
    # table) and a balanced 3-way split of a 32k lane, with and without split-K.
    _decode_case(dev, (1, 4, 64), [65536, 65536 + 64 * 5 + 3, 700], G=8, seed=18, chunk=65536)
    _decode_case(dev, (1, 4, 64), [32769, 10944, 5], G=8, seed=19, chunk=10944)


def test_decode_head_split(dev):
    # One kv head per workgroup, the chunk split over four waves and merged in
    # LDS: single-chunk lanes (output written directly), lanes with split-K
    # partials, quarters that are empty or end in a tail, and G = 16 / G = 1.
    S = dev.DECODE_HEAD_SPLIT
    _decode_case(dev, (2, 4, 64), [1, 5, 64, 65, 200, 256, 257, 1000], G=8, seed=20, chunk=1024 | S)
    _decode_case(dev, (1, 4, 64), [32769, 10944, 5, 70000], G=8, seed=21, chunk=32832 | S)
    _decode_case(dev, (2, 2, 64), [130, 700, 3000], G=16, seed=22, chunk=512 | S)
    _decode_case(dev, (2, 8, 64), [70, 333, 4100], G=1, seed=23, chunk=4096 | S)
    # A table that is not 8-aligned takes the generic path in the first wave.
    _decode_case(dev, (2, 4, 64), [17, 200, 3000], G=8, micro_tokens=6, extent_tokens=48, seed=24,
                 uniform_pages=True, chunk=1024 | S)


def test_decode_group_sizes_fast_path(dev):
    _decode_case(dev, (2, 2, 64), [130, 700], G=16, seed=6)
    _decode_case(dev, (2, 8, 64), [70, 333], G=1, seed=7)


def test_decode_generic_head_dim(dev):
    # The reference contract layouts {L=2,H=2,D=8} (tests/cuda/cuda_kv_test.cpp:668) and D=2 GQA.
    _decode_case(dev, (2, 2, 8), [5, 70, 600], G=2, seed=8)
    _decode_case(dev, (2, 1, 2), [3, 12], G=2, seed=9)
    _decode_case(dev, (1, 2, 128), [90, 1500], G=4, seed=10)


def test_decode_unaligned_pages_generic(dev):
    # 6-token pages: tables not 8-aligned take the generic path.
    _decode_case(dev, (2, 4, 64), [17, 200, 3000], G=8, micro_tokens=6, extent_tokens=48, seed=12,
                 uniform_pages=True)


def _exact_score_inputs(rng, T, H, D, G, values):
    """Q and K with one nonzero dim (d = 0), so every score q.k * scale is exact
    in fp32 on both sides; `values(t, h)` gives V rows [D] (float)."""
    inp = np.zeros((1, 2, T, H, D), dtype=np.float32)
    inp[0, 0, :, :, 0] = rng.integers(-6, 7, size=(T, H)) * 0.5        # k_t[0]
    inp[0, 0, rng.integers(0, T), :, 0] = 8.0                            # a dominant key
    for t in range(T):
        for h in range(H):
            inp[0, 1, t, h] = values(t, h)
    q = np.zeros((H * G, D), dtype=np.float32)
    q[:, 0] = rng.integers(1, 9, size=H * G) * 0.5                       # scores up to 8 * 4 / 8
    return inp.astype(np.float16).view(np.uint16), q.astype(np.float16).view(np.uint16).reshape(-1)


def _decode_fixed(dev, lanes_inputs, H, D, G, chunk=None):
    """Decodes lanes given as (input codes [1][2][T][H][D], query codes) and returns
    (outputs, oracle fp32 references)."""
    QH = H * G
    counts = [inp.shape[2] for inp, _ in lanes_inputs]
    micro_cap = sum(t // 8 + 2 for t in counts) + 8
    ext_cap = sum(t // 64 + 1 for t in counts) + 2
    storage = dev.Storage(1, H, D, micro_cap, ext_cap)
    pools = oracle.HostPools(1, H, D, micro_cap, ext_cap)
    alloc = helpers.SlotAllocator(micro_cap, ext_cap, seed=len(counts))
    lanes, keep = [], []
    for inp, q in lanes_inputs:
        T = inp.shape[2]
        table = helpers.hetero_table(T, alloc)
        keep.append(_populate(dev, storage, pools, table, inp))
        lanes.append((table, T, 0, q, 0.125))
    outs, _, _ = _run_decode(dev, storage, lanes, QH, chunk=chunk)
    refs = [pools.paged_decode(t, T, 0, QH, q, scale, f32=True) for (t, T, _, q, scale) in lanes]
    return outs, refs


def test_decode_constant_value_lanes_return_value_exactly(dev):
    """softmax weights sum to one: a lane whose V rows are all equal must return
    that row bit-exactly, for any scores, chunking and merge path."""
    rng = np.random.default_rng(31)
    H, D, G = 4, 64, 8
    rows = (rng.uniform(-4, 4, size=(H, D))).astype(np.float16).astype(np.float32)
    lanes = []
    for T in [1, 2, 5, 8, 9, 64, 100, 1000, 4000, 9000]:
        lanes.append(_exact_score_inputs(rng, T, H, D, G, lambda t, h: rows[h]))
    for chunk in [None, 1024, 2048 | dev.DECODE_HEAD_SPLIT]:
        outs, _ = _decode_fixed(dev, lanes, H, D, G, chunk=chunk)
        want = np.repeat(rows, G, axis=0).astype(np.float16).view(np.uint16).reshape(-1)
        for (inp, _), got in zip(lanes, outs):
            assert np.array_equal(got, want), (inp.shape[2], chunk, np.abs(helpers.to_f32(got) - helpers.to_f32(want)).max())


def test_decode_near_cancelling_values_dominant_weight(dev):
    """|v| at the generator's bound (4), V rows chosen so that the weighted sum
    of each dim nearly cancels for one query head of the group, one dominant
    key: the output must stay within one fp16 ulp (+1e-5) of the fp32 oracle
    (fp16-rounded weights would be off by up to 4 * 2^-11), and within the
    decode tolerance 2e-3 + 1e-3*|ref|."""
    rng = np.random.default_rng(32)
    H, D, G = 4, 64, 8
    lanes = []
    for trial in range(24):
        T = 2 + trial % 7
        inp, q = _exact_score_inputs(rng, T, H, D, G, lambda t, h: np.zeros(D))
        k0 = helpers.to_f32(inp[0, 0, :, :, 0])                            # [T][H]
        q0 = helpers.to_f32(q.reshape(H * G, D)[:, 0])
        v = rng.choice([-4.0, 4.0], size=(T, H, D)) * rng.uniform(0.9, 1.0, size=(T, H, D))
        for h in range(H):
            s = q0[h * G] * k0[:, h] * 0.125
            w = np.exp(s - s.max())
            w /= w.sum()
            last = int(np.argmin(w))
            rest = np.delete(np.arange(T), last)
            v[last, h] = np.clip(-(w[rest, None] * v[rest, h]).sum(0) / w[last], -4.0, 4.0)
        vals = v.astype(np.float16).astype(np.float32)
        inp_f = helpers.to_f32(inp).reshape(1, 2, T, H, D).copy()
        inp_f[0, 1] = vals
        lanes.append((inp_f.astype(np.float16).view(np.uint16), q))
    outs, refs = _decode_fixed(dev, lanes, H, D, G)
    worst = 0.0
    for got, ref in zip(outs, refs):
        helpers.assert_attention_close(got, ref)
        g = helpers.to_f32(got)
        ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float32)
        err = np.abs(g - ref)
        assert np.all(err <= ulp + 1e-5), float((err - ulp).max())
        worst = max(worst, float(err.max()))
    print(f"near-cancelling decode: max |err| {worst:.2e}", flush=True)


def test_invalid_items_are_reported_not_run(dev):
    """Jobs and items the kernels reject (bad layer index, a multi-chunk lane
    with no workspace, a slot the storage does not hold, a null output) are
    skipped, leave their outputs untouched, and set their bit in the storage's
    fault word, which kimkv_storage_faults returns as KIMKV_INVALID_ARGUMENT
    and clears; valid lanes of the same launch are unaffected."""
    L, H, D, G = 2, 4, 64, 8
    QH = H * G
    storage = dev.Storage(L, H, D, 64, 64)
    pools = oracle.HostPools(L, H, D, 64, 64)
    assert storage.faults() == (0, 0)
    alloc = helpers.SlotAllocator(64, 64, seed=40)
    T = 3000
    table = helpers.hetero_table(T, alloc)
    keep = [_populate(dev, storage, pools, table, _input(L, H, D, T, seed=41))]
    q = oracle.synth_rows(QH * D, 42, 0, D)
    dbuf, qbuf = dev.upload(table), dev.upload(q)
    chunk = 1024                                    # 3 chunks per lane: split-K partials needed
    n = (T + chunk - 1) // chunk
    ws = dev.DeviceBuffer(dev.workspace_bytes(T, chunk, QH, D))
    sentinel = np.full(QH * D, 0x7E00, dtype=np.uint16)              # fp16 NaN
    outs = [dev.upload(sentinel) for _ in range(3)]
    items = np.zeros(3, dtype=dev.DECODE_ITEM)
    items[0] = (dbuf.ptr, len(table), T, 1, qbuf.ptr, ws.ptr, outs[0].ptr, 0.125)   # valid
    items[1] = (dbuf.ptr, len(table), T, L, qbuf.ptr, ws.ptr, outs[1].ptr, 0.125)   # layer out of range
    items[2] = (dbuf.ptr, len(table), T, 0, qbuf.ptr, 0, outs[2].ptr, 0.125)        # no workspace
    prefix = np.array([0, n, 2 * n, 3 * n], dtype=np.uint32)
    ibuf, pbuf = dev.upload(items), dev.upload(prefix)
    storage.decode_launch(ibuf.ptr, pbuf.ptr, 3, 3 * n, chunk, QH)
    status, bits = storage.faults()
    assert status == 1 and bits == dev.FAULT_DECODE_ITEM, (status, bits)
    assert storage.faults() == (0, 0)                                  # cleared
    got = [dev.download(o.ptr, (QH * D,), np.uint16) for o in outs]
    helpers.assert_attention_close(got[0], pools.paged_decode(table, T, 1, QH, q, 0.125, f32=True))
    assert np.array_equal(got[1], sentinel) and np.array_equal(got[2], sentinel)

    # Append: a job naming layer L and one naming a slot past the pool.
    src = dev.upload(np.zeros(2 * H * D, dtype=np.uint16))
    jobs = np.zeros(2, dtype=dev.APPEND_JOB)
    jobs[0] = (src.ptr, src.ptr + 2 * H * D, 0, H * D, L, 1, 1, 5, 0, 0, 0, 0, 0)
    jobs[1] = (src.ptr, src.ptr + 2 * H * D, 0, H * D, 0, 1, 1, 64, 0, 0, 0, 0, 0)
    storage.append_batch(jobs)
    assert storage.faults() == (1, dev.FAULT_APPEND_JOB)
    # Promotion: a micro slot the storage does not hold.
    pj = np.zeros(1, dtype=dev.PROMOTION_JOB)
    pj[0]["micro_slots"] = [1, 2, 3, 4, 5, 6, 7, 64]
    pj[0]["extent_slot"] = 9
    storage.promote_batch(pj)
    assert storage.faults() == (1, dev.FAULT_PROMOTION_JOB)
    # The pages the rejected jobs named are unchanged.
    assert np.array_equal(storage.gather(table, T), pools.gather(table, T))

    # Prefill: an item with a null output.
    per, pre, total = storage.prefill_plan([20], QH)
    pq = dev.upload(oracle.synth_rows(20 * QH * D, 43, 0, D))
    pitems = np.zeros(1, dtype=dev.PREFILL_ITEM)
    pitems[0] = (dbuf.ptr, len(table), T, 20, 0, pq.ptr, 0, 0.125)
    pib, ppb = dev.upload(pitems), dev.upload(pre)
    storage.prefill_launch(pib.ptr, ppb.ptr, 1, total, QH)
    assert storage.faults() == (1, dev.FAULT_PREFILL_ITEM)
    del keep


def test_fill_kv_block_matches_oracle(dev):
    """kimkv_fill_kv: [L][2][T][cols] block with rows synth_kv_row(stream, l, c, token0 + t)."""
    L, T, cols, seed, sid, t0 = 3, 37, 96, 99, 5, 1000
    buf = dev.DeviceBuffer(L * 2 * T * cols * 2)
    dev.fill_kv(buf.ptr, L, T, cols, seed, sid, t0)
    dev.sync()
    got = dev.download(buf.ptr, (L, 2, T, cols), np.uint16)
    for l in range(L):
        for c in range(2):
            want = oracle.synth_rows(T * cols, seed, oracle.kv_row(sid, l, c, t0), cols).reshape(T, cols)
            assert np.array_equal(got[l, c], want)


# ---- chunked prefill ---------------------------------------------------------------

def _prefill_case(dev, shape, cases, G, micro_tokens=8, extent_tokens=64, seed=21, uniform_pages=False,
                  q_gain=1.0):
    """cases: list of (T0, n): a table of T0 + n tokens whose last n are the chunk.  Every new token's
    output must match the oracle's decode of the first T0 + i + 1 tokens with that token's query.
    q_gain scales the queries (larger scores, sharper softmax).  Returns the worst error."""
    L, H, D = shape
    QH = H * G
    totals = [t0 + n for t0, n in cases]
    micro_cap = sum(t // micro_tokens + 2 for t in totals) + 8
    ext_cap = sum(t // extent_tokens + 1 for t in totals) + 2
    storage = dev.Storage(L, H, D, micro_cap, ext_cap, micro_tokens, extent_tokens)
    pools = oracle.HostPools(L, H, D, micro_cap, ext_cap, micro_tokens, extent_tokens)
    alloc = helpers.SlotAllocator(micro_cap, ext_cap, seed=seed, micro_tokens=micro_tokens,
                                  extent_tokens=extent_tokens)
    per, prefix, total = storage.prefill_plan([n for _, n in cases], QH)
    items = np.zeros(len(cases), dtype=dev.PREFILL_ITEM)
    keep, outs, lanes = [], [], []
    scale = 1.0 / math.sqrt(D)
    for i, (t0, n) in enumerate(cases):
        T = t0 + n
        table = helpers.uniform_table(T, micro_tokens, alloc) if uniform_pages else helpers.hetero_table(T, alloc)
        inp = _input(L, H, D, T, seed=seed * 100 + i)
        keep.append(_populate(dev, storage, pools, table, inp))
        q = oracle.synth_rows(n * QH * D, seed * 1000 + i, 0, D)
        if q_gain != 1.0:
            q = (helpers.to_f32(q) * q_gain).astype(np.float16).view(np.uint16)
        layer = (i * 5) % L
        dbuf, qbuf = dev.upload(table), dev.upload(q)
        obuf = dev.DeviceBuffer(n * QH * D * 2)
        items[i] = (dbuf.ptr, len(table), T, n, layer, qbuf.ptr, obuf.ptr, scale)
        keep += [dbuf, qbuf]
        outs.append(obuf)
        lanes.append((table, t0, n, layer, q))
    ibuf, pbuf = dev.upload(items), dev.upload(prefix)
    storage.prefill_launch(ibuf.ptr, pbuf.ptr, len(cases), total, QH)
    # The same batch as an ordered launch (kimkv_prefill_order placement) into
    # second output buffers: the placement must not change a single bit.
    items2 = items.copy()
    outs2 = [dev.DeviceBuffer(n * QH * D * 2) for _, n in cases]
    for i, ob in enumerate(outs2):
        items2[i]["output"] = ob.ptr
    order = dev.prefill_order(H, D, QH, storage.info().compute_units, totals, [n for _, n in cases])
    ibuf2, obuf_order = dev.upload(items2), dev.upload(order)
    storage.prefill_ordered_launch(ibuf2.ptr, len(cases), obuf_order.ptr, len(order), QH)
    dev.sync()
    worst = 0.0
    for (table, t0, n, layer, q), obuf, obuf2 in zip(lanes, outs, outs2):
        got = dev.download(obuf.ptr, (n, QH * D), np.uint16)
        assert np.array_equal(got, dev.download(obuf2.ptr, (n, QH * D), np.uint16)), "ordered launch differs"
        for i in range(n):
            want = pools.paged_decode(table, t0 + i + 1, layer, QH, q[i * QH * D:(i + 1) * QH * D], scale, f32=True)
            worst = max(worst, helpers.assert_attention_close(got[i], want))
    print(f"prefill shape={shape} G={G} cases={cases} per_block={per} blocks={total} ordered={len(order)} "
          f"q_gain={q_gain} max_err={worst:.2e}", flush=True)
    return worst


def test_prefill_causal_matches_per_token_decode(dev):
    """TinyLlama GQA (G=8): chunks at the start of a context, after micro and extent pages, ragged."""
    _prefill_case(dev, (2, 4, 64), [(0, 1), (0, 37), (100, 64), (1000, 200), (5, 7), (64, 130)], G=8)


def test_prefill_group_sizes(dev):
    _prefill_case(dev, (2, 4, 64), [(30, 50), (200, 17)], G=1, seed=22)
    _prefill_case(dev, (2, 2, 64), [(70, 33), (0, 20)], G=4, seed=23)
    _prefill_case(dev, (2, 2, 64), [(129, 40)], G=16, seed=24)


def test_prefill_long_context_segments(dev):
    """Keys beyond one 8192-token group-table segment."""
    _prefill_case(dev, (1, 4, 64), [(9000, 40)], G=8, seed=25)


def test_prefill_sharp_softmax_stays_in_tolerance(dev):
    """Queries scaled 3x and 6x (scores up to ~6x the generator's; the reference point moves often and
    one key dominates many rows): the fast path's queries carry scale * log2(e) in fp16, one more
    rounding per query element than the oracle's fp32 scaling, and its outputs must still be within
    2e-3 + 1e-3 * |ref| of the fp32 oracle."""
    for gain, seed in ((3.0, 29), (6.0, 30)):
        _prefill_case(dev, (2, 4, 64), [(300, 64), (1000, 200), (0, 48)], G=8, seed=seed, q_gain=gain)


def test_prefill_generic_paths(dev):
    _prefill_case(dev, (2, 2, 128), [(90, 20)], G=2, seed=26)                 # D != 64
    _prefill_case(dev, (2, 1, 64), [(50, 9)], G=3, seed=27)                   # G does not divide 16
    _prefill_case(dev, (2, 4, 64), [(17, 30)], G=8, micro_tokens=6, extent_tokens=48, seed=28,
                  uniform_pages=True)                                          # unaligned pages
