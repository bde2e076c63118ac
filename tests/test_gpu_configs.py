"""GPU parity at the benchmark workloads' own sizes.

* config 1: one TinyLlama layer, 4 lanes {17, 100, 513, 1000} in 512-slot
  permuted pools, reserve -> write -> attend through the engine (lane 4
  allocates a new micro page), decode vs the oracle and pages bit-exact;
* config 2a: 64 ragged lanes U[1, 4096] x 22 layers in permuted pools, one
  token appended per lane per layer with tail-page allocation (HipKvCache
  appendBatch), sampled lanes gathered bit-exact against the generator;
* config 2b: one 16 384-token sequence x 22 layers in mixed pages gathered
  bit-exact;
* config 3: 32 lanes log-uniform [128, 8192], 8 groups of 4 forking a
  2048 + r prefix (partial micro tail, copy-on-write), one decode step of 22
  layers through LaneBatch, every lane at layers 0 and 21 vs the oracle, and
  the committed tables (shared prefix pages, distinct COW targets);
* config 4: 256 lanes x 32 768 tokens x 22 layers (189 GB of extent pages)
  through two lane groups on two streams, two decode steps, sampled lanes at
  layers 0 and 21 vs the oracle, tail pages bit-exact;
* config 5: the TinyLlama-1.1B-shaped runner (22 layers, hidden 2048,
  vocab 32 000) on a 16-token chunk plus decode steps beside a second
  request's chunk, logits within 0.035 of the oracle's CPU forward; and the
  config's own workload, the iteration scheduler mixing 4 requests in
  512-token chunked prefill with 60 decode lanes, with per-iteration
  properties and logits at sampled positions against the oracle.

Scenarios after tests/cuda/cuda_kv_test.cpp:287-391,
tests/cuda/cuda_engine_kv_backend_test.cpp:258-345 and
tests/cuda/cuda_model_runner_test.cpp:445-560."""
import math
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle
from tests.helpers import assert_attention_close

pytestmark = pytest.mark.gpu

H, D, QH = 4, 64, 32
HD, QD = H * D, QH * D
THREADS = min(16, os.cpu_count() or 1)


@pytest.fixture(scope="module")
def host(kimkv, dev):
    import importlib
    return importlib.import_module(kimkv.__name__ + ".host")


def _history(seed, sid_of, layers, T):
    """[len(layers)][2][T][H][D] generator rows: token t of the lane is row
    kv_row(sid_of(t), layer, comp, t) (a forked prefix has its root's stream)."""
    out = np.empty((len(layers), 2, T, H, D), dtype=np.uint16)
    runs = []
    a = 0
    while a < T:
        sid = sid_of(a)
        b = a + 1
        while b < T and sid_of(b) == sid:
            b += 1
        runs.append((sid, a, b))
        a = b

    def fill(job):
        li, l, c = job
        for sid, a, b in runs:
            out[li, c, a:b] = oracle.synth_rows((b - a) * HD, seed, oracle.kv_row(sid, l, c, a), HD).reshape(b - a, H, D)

    with ThreadPoolExecutor(THREADS) as pool:
        list(pool.map(fill, [(li, l, c) for li, l in enumerate(layers) for c in range(2)]))
    return out


def _oracle_decode(kv_layer, T, q):
    """fp32-accumulated GQA decode of [2][T][H][D] by the oracle (8-token pages)."""
    pages = (T + 7) // 8
    pools = oracle.HostPools(1, H, D, pages, 1)
    table = np.zeros(pages, dtype=oracle.DESC)
    kv = kv_layer[None]
    for k in range(pages):
        n = min(8, T - 8 * k)
        table[k] = (k, 1, 8 * k, n, 8, 0)
        pools.append_tokens(kv, T, 8 * k, 0, k, 0, n)
    return pools.paged_decode(table, T, 0, QH, q, 1.0 / math.sqrt(D), f32=True)


def _gather_engine(host, dev, engine, rid, L, T):
    """Gathers a request's pages through its committed block table (kimkv_gather on the engine's storage)."""
    _, entries = engine.block_table(rid)
    desc = host.descriptors_from_entries(entries)
    d = dev.upload(desc)
    out = dev.DeviceBuffer(L * 2 * T * HD * 2)
    import ctypes
    dev.check(dev.lib().kimkv_gather(ctypes.c_void_p(engine.storage_handle()), ctypes.c_void_p(d.ptr), len(desc), T,
                                     ctypes.c_void_p(out.ptr), None), "gather")
    return dev.download(out.ptr, (L, 2, T, H, D), np.uint16)


# ---- config 1 ------------------------------------------------------------------------------------------------

def test_config1_engine_append_then_attend(host, dev):
    L, seed = 1, 2024
    contexts = [17, 100, 513, 1000]
    engine = host.Engine(L, H, D, QH, 1 << 16, 512, 512)
    assert engine.permute_free_slots(1, 5) == 0 and engine.permute_free_slots(0, 6) == 0
    stream = dev.Stream()
    stage = dev.DeviceBuffer(L * 2 * 1000 * HD * 2)
    for i, T in enumerate(contexts):
        assert engine.create_request(i + 1) == 0
        dev.fill_kv(stage.ptr, L, T, HD, seed, i, 0, stream)
        rc, _ = engine.append_prefill(i + 1, T, stage.ptr, stream, promote=True)
        assert rc == 0
    # Tokens < 64 in micro pages, the rest in extents (every full 64-token run promoted).
    before = {}
    for i, T in enumerate(contexts):
        _, entries = engine.block_table(i + 1)
        assert [e[2] for e in entries] == [1] * (T // 64) + [0] * ((T % 64 + 7) // 8), (T, entries)
        before[i] = entries
    lanes = len(contexts)
    lane = np.arange(lanes, dtype=np.uint64)
    newkv = dev.DeviceBuffer(lanes * 2 * HD * 2)
    query = dev.DeviceBuffer(lanes * QD * 2)
    out = dev.DeviceBuffer(lanes * QD * 2)
    qseed = seed ^ 0x51
    for i, T in enumerate(contexts):
        dev.fill_kv(newkv.ptr + i * 2 * HD * 2, L, 1, HD, seed, i, T, stream)
        dev.fill_rows(query.ptr + i * QD * 2, QD, qseed, dev.synth_kv_row(i, 0, 0, T), QD, stream)
    ws = dev.DeviceBuffer(lanes * (1 << 16))
    b = host.LaneBatch(engine, lane + np.uint64(1), ws.ptr + lane * np.uint64(1 << 16), 1 << 16, 0.125, stream)
    b.keys[0, :] = newkv.ptr + np.uint64(2 * HD) * (lane * np.uint64(2))
    b.values[0, :] = newkv.ptr + np.uint64(2 * HD) * (lane * np.uint64(2) + np.uint64(1))
    b.queries[0, :] = query.ptr + np.uint64(2 * QD) * lane
    b.outputs[0, :] = out.ptr + np.uint64(2 * QD) * lane
    b.reserve(np.array(contexts, dtype=np.uint32))
    b.write(0)
    b.attend(0)
    b.commit()
    assert not b.failed(), b.status
    assert engine.check_invariants()
    got = dev.download(out.ptr, (lanes, QD), np.uint16)
    used = {(e[2], e[3]) for entries in before.values() for e in entries}
    for i, T in enumerate(contexts):
        _, entries = engine.block_table(i + 1)
        last = entries[-1]
        if T % 8 == 0:            # full tail (lane 4: 1000 = 15 extents + 5 full micro pages): a new micro page
            assert len(entries) == len(before[i]) + 1 and last[:3] == (T, 1, 0)
            assert (last[2], last[3]) not in used
        else:                     # partial micro tail grows in place
            assert len(entries) == len(before[i]) and last[3] == before[i][-1][3]
        hist = _history(seed, lambda t, i=i: i, [0], T + 1)
        assert np.array_equal(_gather_engine(host, dev, engine, i + 1, L, T + 1), hist)
        q = oracle.synth_rows(QD, qseed, oracle.kv_row(i, 0, 0, T), QD)
        assert_attention_close(got[i], _oracle_decode(hist[0], T + 1, q))
    stream.destroy()


# ---- config 2 ------------------------------------------------------------------------------------------------

def test_config2_ragged_append_with_tail_allocation(host, dev):
    L, lanes, seed, steps = 22, 64, 4242, 2
    rng = np.random.default_rng(seed)
    lengths = rng.integers(1, 4097, lanes)
    n_ext = int(sum(lengths // 64)) + 16
    n_micro = 512 + lanes * 12
    cache = host.Cache(L, H, D, n_micro, n_ext)
    assert cache.permute_free_slots(1, seed) == 0 and cache.permute_free_slots(0, seed + 1) == 0
    stream = dev.Stream()
    stage = dev.DeviceBuffer(L * 2 * 4096 * HD * 2)
    for i in range(lanes):
        assert cache.create_request(i + 1) == 0
        n = int(lengths[i])
        dev.fill_kv(stage.ptr, L, n, HD, seed, i, 0, stream)
        r = cache.append(i + 1, n, stage.ptr, stream)
        assert r.ok(), (r.metadata_error, r.device_status)
        for b in range(0, n - n % 64, 64):
            r = cache.promote(i + 1, b, stream)
            assert r.ok(), (i, b)
    per = L * 2 * HD
    newkv = dev.DeviceBuffer(lanes * steps * per * 2)
    for i in range(lanes):
        for s in range(steps):
            dev.fill_kv(newkv.ptr + 2 * (i * steps + s) * per, L, 1, HD, seed, i, int(lengths[i]) + s, stream)
    stream.synchronize()
    ids = np.arange(1, lanes + 1, dtype=np.uint64)
    results = (host.CacheResult * lanes)()
    before = {i: cache.block_table(i + 1)[1] for i in range(lanes)}
    allocating = [i for i in range(lanes) if lengths[i] % 8 == 0]
    assert allocating, "the seeded lengths must include full tails"
    for s in range(steps):
        inputs = newkv.ptr + np.uint64(2 * per) * (np.arange(lanes, dtype=np.uint64) * np.uint64(steps) + np.uint64(s))
        cache.append_batch(ids, 1, inputs, results, stream)
        assert all(results[k].ok() for k in range(lanes)), [(results[k].metadata_error, results[k].device_status)
                                                             for k in range(lanes) if not results[k].ok()][:3]
    assert cache.check_invariants()
    for i in range(lanes):
        entries = cache.block_table(i + 1)[1]
        assert entries[-1][0] + entries[-1][1] == lengths[i] + steps
        if i in allocating:       # the first appended token needed a new micro page
            assert len(entries) == len(before[i]) + 1 and entries[-1][:3] == (int(lengths[i]), steps, 0)
    sample = sorted(set(allocating[:6]) | set(int(x) for x in rng.choice(lanes, 10, replace=False)))
    for i in sample:
        T = int(lengths[i]) + steps
        out = dev.DeviceBuffer(L * 2 * T * HD * 2)
        r = cache.gather(i + 1, out.ptr, stream)
        assert r.ok()
        got = dev.download(out.ptr, (L, 2, T, H, D), np.uint16, stream)
        assert np.array_equal(got, _history(seed, lambda t, i=i: i, list(range(L)), T)), i
    print(f"config 2a: {lanes} lanes, {len(allocating)} allocated tail pages, {len(sample)} lanes gathered bit-exact",
          flush=True)
    cache.close()
    stream.destroy()


def test_config2_gather_16384_tokens_22_layers(host, dev):
    L, T, seed = 22, 16384, 99
    cache = host.Cache(L, H, D, T // 8 + 64, 300)      # the bulk append fills micro pages before promotion
    assert cache.permute_free_slots(1, seed) == 0 and cache.permute_free_slots(0, seed + 1) == 0
    stream = dev.Stream()
    stage = dev.DeviceBuffer(L * 2 * T * HD * 2)
    assert cache.create_request(1) == 0
    dev.fill_kv(stage.ptr, L, T, HD, seed, 7, 0, stream)
    r = cache.append(1, T, stage.ptr, stream)
    assert r.ok()
    for b in range(0, T - 64, 64):            # the last 64 tokens stay in 8 micro pages: a mixed table
        assert cache.promote(1, b, stream).ok()
    kinds = [e[2] for e in cache.block_table(1)[1]]
    assert kinds == [1] * 255 + [0] * 8
    out = dev.DeviceBuffer(L * 2 * T * HD * 2)
    assert cache.gather(1, out.ptr, stream).ok()
    got = dev.download(out.ptr, (L, 2, T, H, D), np.uint16, stream)
    assert np.array_equal(got, dev.download(stage.ptr, (L, 2, T, H, D), np.uint16, stream))
    layers = [0, 11, 21]
    assert np.array_equal(got[layers], _history(seed, lambda t: 7, layers, T))
    cache.close()
    stream.destroy()


# ---- config 3 ------------------------------------------------------------------------------------------------

def test_config3_shared_prefix_fork_cow_decode(host, dev):
    """Groups 0-6 append their own tokens after the fork (the first copies the
    partial prefix page); group 7's lanes hold only the prefix, so the decode
    step's token transaction does the copy-on-write in its per-layer write."""
    L, seed, groups, per_group = 22, 31337, 8, 4
    lanes = groups * per_group
    rng = np.random.default_rng(seed)
    prefix = 2048 + rng.integers(1, 8, groups)
    lengths = np.exp(rng.uniform(np.log(128), np.log(8192), lanes)).astype(np.int64)
    for g in range(groups):
        sl = slice(g * per_group, (g + 1) * per_group)
        lengths[sl] = np.maximum(lengths[sl], prefix[g] + 8) if g < groups - 1 else prefix[g]
    n_ext = int(sum(lengths // 64)) + 32
    engine = host.Engine(L, H, D, QH, 1 << 16, 2048, n_ext)
    assert engine.permute_free_slots(1, seed) == 0 and engine.permute_free_slots(0, seed + 1) == 0
    stream = dev.Stream()
    stage = dev.DeviceBuffer(L * 2 * int(lengths.max()) * HD * 2)
    root_sid = 200
    prefix_tables = {}
    for g in range(groups):
        root = 10_000 + g
        P = int(prefix[g])
        assert engine.create_request(root) == 0
        dev.fill_kv(stage.ptr, L, P, HD, seed, root_sid + g, 0, stream)
        rc, _ = engine.append_prefill(root, P, stage.ptr, stream, promote=True)
        assert rc == 0
        prefix_tables[g] = engine.block_table(root)[1]
        for j in range(per_group):
            i = g * per_group + j
            assert engine.fork_request(root, i + 1) == 0
            n = int(lengths[i]) - P
            if n > 0:
                dev.fill_kv(stage.ptr, L, n, HD, seed, i, P, stream)
                rc, _ = engine.append_prefill(i + 1, n, stage.ptr, stream, promote=True)
                assert rc == 0
        assert engine.release_request(root) == 0
    assert engine.check_invariants()
    lane = np.arange(lanes, dtype=np.uint64)
    newkv = dev.DeviceBuffer(lanes * L * 2 * HD * 2)
    query = dev.DeviceBuffer(lanes * L * QD * 2)
    out = dev.DeviceBuffer(lanes * L * QD * 2)
    qseed = seed ^ 0x5155
    for i in range(lanes):
        T = int(lengths[i])
        dev.fill_kv(newkv.ptr + i * L * 2 * HD * 2, L, 1, HD, seed, i, T, stream)
        for l in range(L):
            dev.fill_rows(query.ptr + (i * L + l) * QD * 2, QD, qseed, dev.synth_kv_row(i, l, 0, T), QD, stream)
    ws_lane = max(dev.workspace_bytes(int(lengths.max()) + 1, 256, QH, D), 256)
    ws = dev.DeviceBuffer(ws_lane * lanes)
    b = host.LaneBatch(engine, lane + np.uint64(1), ws.ptr + lane * np.uint64(ws_lane), ws_lane, 0.125, stream)
    for l in range(L):
        b.keys[l, :] = newkv.ptr + np.uint64(2 * HD) * (lane * np.uint64(2 * L) + np.uint64(2 * l))
        b.values[l, :] = newkv.ptr + np.uint64(2 * HD) * (lane * np.uint64(2 * L) + np.uint64(2 * l + 1))
        b.queries[l, :] = query.ptr + np.uint64(2 * QD) * (lane * np.uint64(L) + np.uint64(l))
        b.outputs[l, :] = out.ptr + np.uint64(2 * QD) * (lane * np.uint64(L) + np.uint64(l))
    b.reserve(lengths.astype(np.uint32))
    for l in range(L):
        b.write(l)
        b.attend(l)
    b.commit()
    assert not b.failed(), sorted(set(b.status.tolist()))
    assert engine.check_invariants()
    # Tables: the full prefix pages are shared by the group, the partial prefix page was copied per lane.
    for g in range(groups):
        P = int(prefix[g])
        shared = [e for e in prefix_tables[g] if e[0] + e[1] <= P - P % 8]
        tails = set()
        for j in range(per_group):
            entries = engine.block_table(g * per_group + j + 1)[1]
            assert [(e[2], e[3], e[4]) for e in entries[:len(shared)]] == [(e[2], e[3], e[4]) for e in shared]
            tail = next(e for e in entries if e[0] == P - P % 8)
            assert tail[1] > P % 8 and (tail[2], tail[3]) != tuple(prefix_tables[g][-1][2:4])
            tails.add((tail[2], tail[3]))
        assert len(tails) == per_group, (g, tails)
    got = dev.download(out.ptr, (lanes, L, QD), np.uint16)
    worst = 0.0
    for i in range(lanes):
        g = i // per_group
        P = int(prefix[g])
        T = int(lengths[i]) + 1
        hist = _history(seed, lambda t, g=g, i=i, P=P: root_sid + g if t < P else i, [0, L - 1], T)
        for li, l in enumerate([0, L - 1]):
            q = oracle.synth_rows(QD, qseed, oracle.kv_row(i, l, 0, T - 1), QD)
            worst = max(worst, assert_attention_close(got[i, l], _oracle_decode(hist[li], T, q)))
    print(f"config 3: {lanes} lanes, prefixes {[int(p) for p in prefix]}, max decode err {worst:.2e}", flush=True)
    stream.destroy()


# ---- config 4 ------------------------------------------------------------------------------------------------

def test_config4_hbm_scale_two_lane_groups(host, dev):
    """Config 4 at its full size: 256 lanes x 32 768-token contexts x 22 layers (131 072 extent pages,
    189 GB, slots permuted) built by the engine's bulk prefill + promotion, then two decode steps
    through two lane groups of 128 token transactions on two streams, the first group committed after
    the second group's layers are queued (src/cuda/engine/backend.cpp:198-259 at 256 lanes).  Eight
    lanes from both groups at layers 0 and 21 against the oracle's decode of the generator's history
    (32 770 tokens), committed tables (512 extents + one micro tail of two tokens), and two lanes' tail
    pages gathered bit-exact."""
    lanes, context, L, steps, seed = 256, 32768, 22, 2, 4040
    ws_lane = max(dev.workspace_bytes(context + steps, 64, QH, D), 256)
    n_micro = lanes * 2 + 64
    engine = host.Engine(L, H, D, QH, ws_lane, n_micro, lanes * context // 64)
    streams = [dev.Stream(), dev.Stream()]
    try:
        assert engine.permute_free_slots(1, seed) == 0 and engine.permute_free_slots(0, seed + 1) == 0
        stage = dev.DeviceBuffer(L * 2 * 512 * HD * 2)
        for i in range(lanes):
            assert engine.create_request(i + 1) == 0
            for t in range(0, context, 512):
                dev.fill_kv(stage.ptr, L, 512, HD, seed, i, t, streams[0])
                rc, promoted = engine.append_prefill(i + 1, 512, stage.ptr, streams[0], promote=True)
                assert rc == 0 and promoted == 8, (i, t, rc, promoted)
        streams[0].synchronize()
        del stage
        print(f"config 4: {lanes} x {context} tokens prefilled, "
              f"{engine.snapshot().storage_reserved_bytes / 1e9:.1f} GB of pools", flush=True)
        lane = np.arange(lanes, dtype=np.uint64)
        newkv = dev.DeviceBuffer(lanes * L * 2 * steps * HD * 2)       # [lane][layer][comp][step][HD]
        query = dev.DeviceBuffer(lanes * L * steps * QD * 2)           # [lane][layer][step][QD]
        out = dev.DeviceBuffer(lanes * L * QD * 2)                      # [lane][layer][QD]
        qseed = seed ^ 0x5155
        for i in range(lanes):
            for l in range(L):
                for c in range(2):
                    dev.fill_rows(newkv.ptr + (((i * L + l) * 2 + c) * steps) * HD * 2, steps * HD, seed,
                                  dev.synth_kv_row(i, l, c, context), HD)
                dev.fill_rows(query.ptr + ((i * L + l) * steps) * QD * 2, steps * QD, qseed,
                              dev.synth_kv_row(i, l, 0, context), QD)
        dev.sync()
        ws = dev.DeviceBuffer(ws_lane * lanes)
        groups = []
        layer = np.arange(L, dtype=np.uint64)[:, None]
        for g, sl in enumerate([slice(0, lanes // 2), slice(lanes // 2, lanes)]):
            b = host.LaneBatch(engine, lane[sl] + np.uint64(1), ws.ptr + lane[sl] * np.uint64(ws_lane), ws_lane,
                               1.0 / math.sqrt(D), streams[g])
            row = lane[sl][None, :] * np.uint64(L) + layer                    # [layer][lane] (lane, layer) index
            kbase = newkv.ptr + np.uint64(2 * HD) * row * np.uint64(2 * steps)
            qbase = query.ptr + np.uint64(2 * QD) * row * np.uint64(steps)
            b.outputs[:] = out.ptr + np.uint64(2 * QD) * row
            groups.append((b, kbase, qbase))
        pending = None
        for step in range(steps):
            for b, kbase, qbase in groups:
                b.keys[:] = kbase + np.uint64(2 * HD * step)
                b.values[:] = kbase + np.uint64(2 * HD * (steps + step))
                b.queries[:] = qbase + np.uint64(2 * QD * step)
                b.reserve(context + step)
                assert not b.failed(), ("reserve", step, sorted(set(b.status.tolist())))
                for l in range(L):
                    b.write(l)
                    b.attend(l)
                assert not b.failed(), ("launch", step, sorted(set(b.status.tolist())))
                if pending is not None:          # the other group's commit waits behind this group's launches
                    pending.commit()
                    assert not pending.failed()
                pending = b
        pending.commit()
        assert not pending.failed()
        assert engine.check_invariants()
        T = context + steps
        got = dev.download(out.ptr, (lanes, L, QD), np.uint16)
        sample = [0, 37, 90, 127, 128, 171, 200, 255]
        cases = []
        for i in sample:
            hist = _history(seed, lambda t, i=i: i, [0, L - 1], T)
            for li, l in enumerate([0, L - 1]):
                q = oracle.synth_rows(QD, qseed, oracle.kv_row(i, l, 0, context) + steps - 1, QD)
                cases.append((i, l, hist[li], q))
        with ThreadPoolExecutor(THREADS) as pool:
            wants = list(pool.map(lambda c: _oracle_decode(c[2], T, c[3]), cases))
        worst = 0.0
        for (i, l, _, _), want in zip(cases, wants):
            worst = max(worst, assert_attention_close(got[i, l], want))
        # Tables and tail pages.
        for i in (5, 250):
            _, entries = engine.block_table(i + 1)
            assert [e[2] for e in entries] == [1] * 512 + [0] and entries[-1][:2] == (context, steps)
            tail = entries[-3:]                                  # two extents + the micro tail
            base = tail[0][0]
            desc = host.descriptors_from_entries([(e[0] - base,) + tuple(e[1:]) for e in tail])
            d = dev.upload(desc)
            buf = dev.DeviceBuffer(L * 2 * (T - base) * HD * 2)
            import ctypes
            dev.check(dev.lib().kimkv_gather(ctypes.c_void_p(engine.storage_handle()), ctypes.c_void_p(d.ptr),
                                             len(desc), T - base, ctypes.c_void_p(buf.ptr), None), "gather")
            pages = dev.download(buf.ptr, (L, 2, T - base, H, D), np.uint16)
            want = np.empty_like(pages)
            for l in range(L):
                for c in range(2):
                    want[l, c] = oracle.synth_rows((T - base) * HD, seed, oracle.kv_row(i, l, c, base),
                                                   HD).reshape(T - base, H, D)
            assert np.array_equal(pages, want), i
        print(f"config 4: {lanes} lanes x {T} tokens x {L} layers, 2 groups on 2 streams, "
              f"{len(cases)} lane-layers max decode err {worst:.2e}", flush=True)
    finally:
        engine.close()
        for st in streams:
            st.destroy()


# ---- config 5 ------------------------------------------------------------------------------------------------

def test_config5_tinyllama_1b_runner_logits(host, dev):
    from oracle import model as om
    cfg = om.ModelConfig(hidden_size=2048, intermediate_size=5632, layer_count=22, attention_head_count=32,
                         kv_head_count=4, head_dimension=64, vocabulary_size=32000, max_position_embeddings=2048)
    seed, tol = 4321, 0.035
    engine = host.Engine(22, 4, 64, 32, 1 << 16, 256, 16)
    stream = dev.Stream()
    mc = host.ModelConfig(cfg.hidden_size, cfg.intermediate_size, cfg.layer_count, cfg.attention_head_count,
                          cfg.kv_head_count, cfg.head_dimension, cfg.vocabulary_size, cfg.max_position_embeddings,
                          cfg.bos_token_id, cfg.eos_token_id, cfg.rms_norm_epsilon, cfg.rope_theta)
    runner = host.Runner(engine, mc, seed, 64, 4, stream)
    ref_a = om.ReferenceModel(cfg, seed, threads=THREADS)
    ref_b = ref_a.fresh()
    rng = np.random.default_rng(seed)
    pa = [int(t) for t in rng.integers(3, cfg.vocabulary_size, 16)]
    pb = [int(t) for t in rng.integers(3, cfg.vocabulary_size, 9)]
    assert engine.create_request(1) == 0 and engine.create_request(2) == 0
    worst = 0.0

    def check(got, want, tag):
        nonlocal worst
        err = float(np.max(np.abs(got - want)))
        assert err < tol, (tag, err)
        worst = max(worst, err)

    nxt, ok, logits = runner.forward([(1, 0, pa)], want_logits=True)
    assert ok.all()
    for p, t in enumerate(pa):
        want = ref_a.forward(t, p)
    check(logits[0], want, "A chunk")
    ga, pos = int(nxt[0]), len(pa)
    # A decodes while B's prompt goes as a chunk, then both decode.
    nxt, ok, logits = runner.forward([(1, pos, [ga]), (2, 0, pb)], want_logits=True)
    assert ok.all()
    check(logits[0], ref_a.forward(ga, pos), "A decode 1")
    for p, t in enumerate(pb):
        wb = ref_b.forward(t, p)
    check(logits[1], wb, "B chunk")
    for step in range(2):
        ga, gb = int(nxt[0]), int(nxt[1])
        pos += 1
        nxt, ok, logits = runner.forward([(1, pos, [ga]), (2, len(pb) + step, [gb])], want_logits=True)
        assert ok.all()
        check(logits[0], ref_a.forward(ga, pos), f"A decode {step + 2}")
        check(logits[1], ref_b.forward(gb, len(pb) + step), f"B decode {step + 1}")
    assert engine.check_invariants()
    print(f"config 5: TinyLlama-1.1B shape, max logit err {worst:.2e}", flush=True)
    runner.close()
    stream.destroy()


def test_config5_scheduler_chunked_prefill_beside_60_decode_lanes(host, dev):
    """Config 5's own workload: the iteration scheduler over the TinyLlama-1.1B-shaped runner with 60
    decode lanes beside 4 requests in 512-token chunked prefill (prompts U[256, 2048], a finished one
    replaced at once), max_batched_tokens 4 x 512 + 60 (tests/cuda/cuda_model_runner_test.cpp:703-825
    at this shape).  Every iteration of the mix: one model call, every active request one span (decode
    lanes one position further, prefilling requests min(512, remaining) positions), the scheduler's
    token counts matching, each request's committed KV length = its last processed position + 1, engine
    invariants.  Logits (runner watch) against the oracle's CPU forward within 0.035 at: two decode
    lanes (256-token prompts) from their prompt's last row through every decode step, teacher-forced
    with the lanes' own greedy tokens; a 700-token prompt's chunk ends (positions 511 and 699).  The
    drained terminals hold every lane's tokens, all inside the vocabulary."""
    from oracle import model as om
    cfg = om.ModelConfig(hidden_size=2048, intermediate_size=5632, layer_count=22, attention_head_count=32,
                         kv_head_count=4, head_dimension=64, vocabulary_size=32000, max_position_embeddings=2048)
    L, V = cfg.layer_count, cfg.vocabulary_size
    n_dec, n_pre, chunk, max_new, tol = 60, 4, 512, 48, 0.035
    budget = n_pre * chunk + n_dec
    seed = 9090
    rng = np.random.default_rng(seed)
    engine = host.Engine(L, H, D, QH, 1 << 20, (n_dec * 1100 + (2 * n_pre + 4) * 2048) // 8 + 512, 16)
    assert engine.permute_free_slots(0, seed) == 0
    stream = dev.Stream()
    mc = host.ModelConfig(cfg.hidden_size, cfg.intermediate_size, L, cfg.attention_head_count, cfg.kv_head_count,
                          cfg.head_dimension, V, cfg.max_position_embeddings, cfg.bos_token_id, cfg.eos_token_id,
                          cfg.rms_norm_epsilon, cfg.rope_theta)
    runner = host.Runner(engine, mc, seed, budget + 64, n_dec + n_pre + 8, stream)
    sched = host.Scheduler(engine, runner, max_active=n_dec + n_pre + 8, max_batched_tokens=budget,
                           max_kv_tokens=1 << 40, prefill_chunk=chunk)
    prompts = {}

    def submit(rid, n, new):
        prompts[rid] = [int(t) for t in rng.integers(3, V, n)]
        assert sched.submit(rid, prompts[rid], new) == "none"

    sampled = [1, 2]
    for rid in range(1, n_dec + 1):
        submit(rid, 256 if rid in sampled else int(rng.integers(256, 1025)), max_new)
    seen = {rid: {} for rid in sampled}            # rid -> {position: GPU logits}

    def record(rows, pos, cnt, ids):
        for k, rid in enumerate(ids):
            if rid in seen and cnt[k]:
                seen[rid][int(pos[k])] = rows[k].copy()

    # Setup: until every decode lane is decoding.
    setup = 0
    while True:
        rows, pos, cnt = runner.watch_logits(sampled)
        r = sched.run_iteration()
        record(rows, pos, cnt, sampled)
        setup += 1
        assert r.model_forward_batches == 1 and setup < 200
        if r.prefill_tokens == 0:
            break
    assert not sched.take_terminals()
    assert r.decode_tokens == n_dec

    # The mix: 4 prefilling requests (one of them the sampled 700-token prompt) beside the 60 lanes.
    last = {}
    for rid in range(1, n_dec + 1):
        _, entries = engine.block_table(rid)
        last[rid] = entries[-1][0] + entries[-1][1] - 1        # last committed position
    prefilling, next_rid, pre_sample = {}, 101, 101
    mix_iters = 6
    for it in range(mix_iters):
        while len(prefilling) < n_pre:
            n = 700 if next_rid == pre_sample else int(rng.integers(256, 2049))
            submit(next_rid, n, 1)
            prefilling[next_rid] = 0                             # prompt tokens processed
            next_rid += 1
        ids = list(range(1, n_dec + 1)) + sorted(prefilling)
        rows, pos, cnt = runner.watch_logits(ids)
        want_pre = {rid: min(chunk, len(prompts[rid]) - done) for rid, done in prefilling.items()}
        finishing = {rid for rid, n in want_pre.items() if prefilling[rid] + n == len(prompts[rid])}
        r = sched.run_iteration()
        print(f"config 5 mix iteration {it}: prefill {r.prefill_tokens} decode {r.decode_tokens} "
              f"forward {r.model_forward_tokens} terminals {r.terminals_produced}", flush=True)
        assert r.model_forward_batches == 1
        assert r.decode_tokens == n_dec and r.prefill_tokens == sum(want_pre.values())
        assert r.model_forward_tokens == r.prefill_tokens + r.decode_tokens
        assert r.terminals_produced == len(finishing)
        assert list(cnt) == [1] * len(ids), "every active request gets one span per iteration"
        for k, rid in enumerate(ids):
            if rid <= n_dec:
                assert pos[k] == last[rid] + 1, (rid, int(pos[k]), last[rid])
                last[rid] = int(pos[k])
            else:
                assert pos[k] == prefilling[rid] + want_pre[rid] - 1, (rid, int(pos[k]))
                if rid == pre_sample:
                    seen.setdefault(rid, {})[int(pos[k])] = rows[k].copy()
        record(rows, pos, cnt, ids)
        for rid in ids:
            if rid in finishing:
                continue
            _, entries = engine.block_table(rid)
            committed = entries[-1][0] + entries[-1][1]
            want = last[rid] + 1 if rid <= n_dec else prefilling[rid] + want_pre[rid]
            assert committed == want, (rid, committed, want)
        for rid, n in want_pre.items():
            prefilling[rid] += n
        for t in sched.take_terminals():
            assert t["error"] == "none" and t["request_id"] in finishing, t
            assert t["completion_tokens"] == 1 and all(0 <= x < V for x in t["tokens"])
            prefilling.pop(t["request_id"])
        assert engine.check_invariants()
    runner.watch_logits([])
    terminals = {t["request_id"]: t for t in sched.drain()}
    for rid in range(1, n_dec + 1):
        t = terminals[rid]
        assert t["error"] == "none" and t["prompt_tokens"] == len(prompts[rid]), t
        if t["reason"] == "eos_token":      # random weights do produce the model's EOS now and then
            assert t["tokens"][-1] == cfg.eos_token_id and len(t["tokens"]) <= max_new, t
        else:
            assert t["reason"] == "max_new_tokens" and len(t["tokens"]) == max_new, t
        assert all(0 <= x < V for x in t["tokens"])
    sched.close()
    assert engine.snapshot().request_count == 0

    # Oracle: logits at the recorded positions.
    ref = om.ReferenceModel(cfg, seed, threads=THREADS)
    worst = 0.0

    def check(got, want, tag):
        nonlocal worst
        err = float(np.max(np.abs(got - want)))
        assert err < tol, (tag, err)
        worst = max(worst, err)

    for rid in sampled:
        m = ref.fresh()
        P = len(prompts[rid])
        check(seen[rid][P - 1], m.forward_span(prompts[rid], 0), f"lane {rid} prompt")
        toks = terminals[rid]["tokens"]
        positions = sorted(p for p in seen[rid] if p >= P)
        assert positions == list(range(P, P + len(positions))) and len(positions) >= mix_iters
        for p in positions:
            check(seen[rid][p], m.forward(toks[p - P], p), f"lane {rid} position {p}")
    m = ref.fresh()
    pp = prompts[pre_sample]
    assert sorted(seen[pre_sample]) == [511, 699]
    check(seen[pre_sample][511], m.forward_span(pp[:512], 0), "700-token prompt, first chunk")
    check(seen[pre_sample][699], m.forward_span(pp[512:], 512), "700-token prompt, second chunk")
    print(f"config 5 workload: {setup} setup + {mix_iters} mixed iterations, max logit err {worst:.2e}", flush=True)
    runner.close()
    stream.destroy()
