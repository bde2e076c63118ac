"""GPU tests of the C++ host layer over the HIP kernels: the engine backend
(token transactions, batched attention/write, fork + partial-tail COW, fault
injection, engine promotion) and the HipKvCache facade.  Scenarios mirror the
reference's tests/cuda/cuda_engine_kv_backend_test.cpp and
tests/cuda/cuda_kv_test.cpp; every data check is against closed forms or the
oracle."""
import ctypes
import math
import types

import numpy as np
import pytest

import oracle
from tests.helpers import make_kv_closed_form, to_f32

pytestmark = pytest.mark.gpu

SUBMISSION_FAILED = 8   # EngineKvError::SubmissionFailed
EXECUTION_FAILED = 9    # EngineKvError::ExecutionFailed
DEV_SUBMISSION_FAILED = 4
DEV_EXECUTION_FAILED = 6


def f16(*values):
    return np.array(values, dtype=np.float16).view(np.uint16)


@pytest.fixture(scope="module")
def host(kimkv, dev):
    import importlib
    return importlib.import_module(kimkv.__name__ + ".host")


class Buffers:
    """Per-lane device buffers (key/value per layer, query, output, workspace)."""

    def __init__(self, dev, layers=2, kv=2, qh=2, dim=2, workspace=4096):
        self.dev = dev
        self.keys = [dev.DeviceBuffer(kv * dim * 2) for _ in range(layers)]
        self.values = [dev.DeviceBuffer(kv * dim * 2) for _ in range(layers)]
        self.query = dev.DeviceBuffer(qh * dim * 2)
        self.output = dev.DeviceBuffer(qh * dim * 2)
        self.workspace = dev.DeviceBuffer(workspace)
        self.workspace_bytes = workspace


def reference_output(history, new_token):
    """Closed-form GQA output for the engine scenario (cuda_engine_kv_backend_test.cpp:96-130)."""
    tokens = list(history) + [new_token]
    scale = 1.0 / math.sqrt(2.0)
    queries = [(0.5, 0.25), (-0.2, 0.4)]
    out = [0.0] * 4
    for qh in range(2):
        scores = [(queries[qh][0] * (0.1 * (t + 1) + 0.02) + queries[qh][1] * (-0.05 * t + 0.01)) * scale
                  for t in tokens]
        m = max(scores)
        den = sum(math.exp(s - m) for s in scores)
        for t, s in zip(tokens, scores):
            p = math.exp(s - m) / den
            out[2 * qh] += p * (t + 1 + 0.2)
            out[2 * qh + 1] += p * ((t + 1) * 0.5 - 0.1)
    return out


def run_token(host, dev, engine, rid, history, token, buf, stream, fault=None):
    """One decode token through reserve/write/attend/commit (cuda_engine_kv_backend_test.cpp:132-244)."""
    rc, txn = engine.reserve_token(rid, len(history), stream)
    assert rc == 0, host.ENGINE_ERRORS[rc]
    assert engine.snapshot().active_transaction_count == 1
    dev.copy_to_device(buf.query.ptr, f16(0.5, 0.25, -0.2, 0.4), stream)
    if fault == "submission":
        assert engine.inject_failure_once("submission")
    for layer in range(2):
        off = 0.02 if layer == 1 else 0.0
        dev.copy_to_device(buf.keys[layer].ptr, f16(0.1 * (token + 1) + off, -0.05 * token + off * 0.5), stream)
        dev.copy_to_device(buf.values[layer].ptr, f16(token + 1 + off * 10.0, (token + 1) * 0.5 - off * 5.0), stream)
        rc = txn.write_layer(layer, buf.keys[layer].ptr, buf.values[layer].ptr)
        if fault == "submission" and layer == 0:
            assert rc == SUBMISSION_FAILED
            assert txn.rollback() == 0
            assert engine.check_invariants()
            return False
        assert rc == 0, host.ENGINE_ERRORS[rc]
        rc = txn.attend_layer(layer, buf.query.ptr, buf.output.ptr, buf.workspace.ptr, buf.workspace_bytes,
                              1.0 / math.sqrt(2.0))
        assert rc == 0, host.ENGINE_ERRORS[rc]
    if fault == "completion":
        assert engine.inject_failure_once("completion")
        assert txn.commit() == EXECUTION_FAILED
        assert engine.check_invariants()
        return False
    assert txn.commit() == 0
    out = to_f32(dev.download(buf.output.ptr, (4,), np.uint16))
    expected = np.array(reference_output(history, token), dtype=np.float32)
    assert np.all(np.abs(out - expected) < 0.035), (out, expected)
    history.append(token)
    assert engine.check_invariants()
    assert engine.snapshot().active_transaction_count == 0
    return True


def test_engine_backend_tokens_fork_and_faults(host, dev):
    """testBackend(Heterogeneous), cuda_engine_kv_backend_test.cpp:246-345."""
    engine = host.Engine(2, 1, 2, 2, 4096, 32, 4)
    snap = engine.snapshot()
    assert snap.primary_page_tokens == 8 and snap.secondary_page_tokens == 64
    assert snap.primary_page_capacity == 32 and snap.secondary_page_capacity == 4
    assert snap.storage_reserved_bytes != 0
    assert engine.create_request(1) == 0
    stream = dev.Stream()
    buf = Buffers(dev)
    parent = []
    for token in range(10):
        assert run_token(host, dev, engine, 1, parent, token, buf, stream)
    snap = engine.snapshot()
    assert snap.committed_token_count == 10
    assert snap.allocated_primary_pages != 0 and snap.successful_primary_allocations != 0

    assert engine.fork_request(1, 2) == 0
    child = list(parent)
    assert run_token(host, dev, engine, 2, child, 21, buf, stream)   # partial-tail COW
    assert engine.snapshot().committed_token_count == 21

    before = engine.snapshot().committed_token_count
    assert not run_token(host, dev, engine, 1, parent, 30, buf, stream, fault="submission")
    assert engine.snapshot().committed_token_count == before
    assert not run_token(host, dev, engine, 1, parent, 31, buf, stream, fault="completion")
    assert engine.snapshot().committed_token_count == before

    # The parent still decodes correctly after both faults.
    assert run_token(host, dev, engine, 1, parent, 12, buf, stream)
    assert engine.release_request(2) == 0
    assert engine.release_request(1) == 0
    snap = engine.snapshot()
    assert snap.request_count == 0 and snap.committed_token_count == 0
    assert snap.allocated_primary_pages == 0 and snap.allocated_secondary_pages == 0
    assert engine.check_invariants()
    stream.destroy()


def _closed_form_prefill(dev, tokens):
    """[layer][K/V][token][1 head][2 dims] fp16 rows of run_token's closed form for `tokens`."""
    kv = np.zeros((2, 2, len(tokens), 1, 2), dtype=np.float32)
    for layer in range(2):
        off = 0.02 if layer == 1 else 0.0
        for j, t in enumerate(tokens):
            kv[layer, 0, j, 0] = (0.1 * (t + 1) + off, -0.05 * t + off * 0.5)
            kv[layer, 1, j, 0] = (t + 1 + off * 10.0, (t + 1) * 0.5 - off * 5.0)
    return kv.astype(np.float16).view(np.uint16)


def test_engine_device_table_after_rollback_and_append(host, dev):
    """Each request's device block table is patched in place per token; a
    reservation that is rolled back leaves the candidate in the device copy.
    The next reservation must rewrite it, also when a prefill append has
    meanwhile moved the table to the version the abandoned candidate had,
    and when a fork's first token replaces the shared partial tail."""
    engine = host.Engine(2, 1, 2, 2, 4096, 64, 4)
    assert engine.create_request(1) == 0
    stream = dev.Stream()
    buf = Buffers(dev)
    history = []
    for token in range(10):
        assert run_token(host, dev, engine, 1, history, token, buf, stream)
    staged = dev.DeviceBuffer(2 * 2 * 16 * 2 * 2)
    for round_ in range(2):
        # Reserve, write and attend a token, then roll it back.
        rc, txn = engine.reserve_token(1, len(history), stream)
        assert rc == 0, host.ENGINE_ERRORS[rc]
        for layer in range(2):
            assert txn.write_layer(layer, buf.keys[layer].ptr, buf.values[layer].ptr) == 0
            assert txn.attend_layer(layer, buf.query.ptr, buf.output.ptr, buf.workspace.ptr, buf.workspace_bytes,
                                    1.0 / math.sqrt(2.0)) == 0
        assert txn.rollback() == 0
        txn.close()
        assert engine.check_invariants()
        if round_ == 0:
            # Same version as before the reservation: rewritten on the next reserve.
            assert run_token(host, dev, engine, 1, history, 40, buf, stream)
        else:
            # A prefill append takes the table to the abandoned candidate's version.
            tokens = list(range(50, 55))
            dev.copy_to_device(staged.ptr, _closed_form_prefill(dev, tokens).reshape(-1), stream)
            rc, _ = engine.append_prefill(1, len(tokens), staged.ptr, stream, promote=False)
            assert rc == 0, host.ENGINE_ERRORS[rc]
            history.extend(tokens)
            assert run_token(host, dev, engine, 1, history, 41, buf, stream)
    for token in range(42, 48):
        assert run_token(host, dev, engine, 1, history, token, buf, stream)
    # A fork shares the partial tail; its first token replaces it (COW) in
    # the child's own device table while the parent's stays valid.
    assert engine.fork_request(1, 2) == 0
    child = list(history)
    assert run_token(host, dev, engine, 2, child, 60, buf, stream)
    assert run_token(host, dev, engine, 1, history, 61, buf, stream)
    assert run_token(host, dev, engine, 2, child, 62, buf, stream)
    assert engine.release_request(2) == 0
    assert engine.release_request(1) == 0
    assert engine.check_invariants()
    stream.destroy()


def test_extent_plus_micro_attention_known_answer(host, dev):
    """testExtentPagedAttention, cuda_engine_kv_backend_test.cpp:347-500: 64
    tokens K=(1,1), V=(t/64, -t/128) promoted into one extent, then a token
    K=(1,1) V=(1,-1) attended with q=(1,1): uniform weights give
    (0.5, -0.2577)."""
    engine = host.Engine(1, 1, 2, 1, 65 * 4, 9, 1)
    assert engine.create_request(50) == 0
    stream = dev.Stream()
    buf = Buffers(dev, layers=1, kv=1, qh=1, dim=2, workspace=65 * 4)
    dev.copy_to_device(buf.query.ptr, f16(1.0, 1.0), stream)
    for t in range(64):
        rc, txn = engine.reserve_token(50, t, stream)
        assert rc == 0
        dev.copy_to_device(buf.keys[0].ptr, f16(1.0, 1.0), stream)
        dev.copy_to_device(buf.values[0].ptr, f16(t / 64.0, -t / 128.0), stream)
        assert txn.write_layer(0, buf.keys[0].ptr, buf.values[0].ptr) == 0
        assert txn.attend_layer(0, buf.query.ptr, buf.output.ptr, buf.workspace.ptr, buf.workspace_bytes,
                                1.0 / math.sqrt(2.0)) == 0
        assert txn.commit() == 0
    rc, promoted = engine.promote_request(50, stream)
    assert rc == 0 and promoted == 1
    version, entries = engine.block_table(50)
    assert len(entries) == 1 and entries[0][2] == 1   # one extent entry

    rc, txn = engine.reserve_token(50, 64, stream)
    assert rc == 0
    dev.copy_to_device(buf.keys[0].ptr, f16(1.0, 1.0), stream)
    dev.copy_to_device(buf.values[0].ptr, f16(1.0, -1.0), stream)
    assert txn.write_layer(0, buf.keys[0].ptr, buf.values[0].ptr) == 0
    assert txn.attend_layer(0, buf.query.ptr, buf.output.ptr, buf.workspace.ptr, buf.workspace_bytes,
                            1.0 / math.sqrt(2.0)) == 0
    assert txn.commit() == 0
    out = to_f32(dev.download(buf.output.ptr, (2,), np.uint16))
    assert abs(out[0] - 0.5) < 0.01 and abs(out[1] + 0.2577) < 0.01, out
    _, entries = engine.block_table(50)
    assert [e[2] for e in entries] == [1, 0]          # extent then micro
    assert engine.check_invariants()
    assert engine.release_request(50) == 0
    stream.destroy()


def test_batched_attention_failure_isolation(host, dev):
    """testBatchedAttentionFailureIsolation(Heterogeneous), cuda_engine_kv_backend_test.cpp:502-610."""
    engine = host.Engine(1, 1, 2, 2, 4096, 16, 2)
    assert engine.create_request(70) == 0 and engine.create_request(71) == 0
    stream = dev.Stream()
    first, second = Buffers(dev, layers=1, kv=1), Buffers(dev, layers=1, kv=1)
    rc1, t1 = engine.reserve_token(70, 0, stream)
    rc2, t2 = engine.reserve_token(71, 0, stream)
    assert rc1 == 0 and rc2 == 0
    for b, k, v in ((first, (0.1, 0.2), (1.0, 2.0)), (second, (0.3, 0.4), (3.0, 4.0))):
        dev.copy_to_device(b.query.ptr, f16(0.5, 0.25, -0.2, 0.4), stream)
        dev.copy_to_device(b.keys[0].ptr, f16(*k), stream)
        dev.copy_to_device(b.values[0].ptr, f16(*v), stream)
    assert t1.write_layer(0, first.keys[0].ptr, first.values[0].ptr) == 0
    assert t2.write_layer(0, second.keys[0].ptr, second.values[0].ptr) == 0
    assert engine.inject_failure_once("submission")
    scale = 1.0 / math.sqrt(2.0)
    st = host.attend_layer_batch(
        [t1, t2], [(0, b.query.ptr, b.output.ptr, b.workspace.ptr, 4096, scale) for b in (first, second)])
    assert st[0] == SUBMISSION_FAILED
    assert st[1] == 0
    assert t1.rollback() == 0
    assert t2.commit() == 0
    out = to_f32(dev.download(second.output.ptr, (4,), np.uint16))
    np.testing.assert_allclose(out, [3.0, 4.0, 3.0, 4.0], atol=0.01)
    snap = engine.snapshot()
    assert snap.committed_token_count == 1 and snap.active_transaction_count == 0
    assert snap.batched_attention_submissions == 1 and snap.batched_attention_lanes == 1
    assert engine.release_request(71) == 0 and engine.release_request(70) == 0
    assert engine.check_invariants()
    stream.destroy()


def _oracle_lane(history_kv, layer, q_codes, qh, kv, dim, scale):
    """fp32 GQA over a lane's full history for one layer; history_kv[t] = (K[kv][dim], V[kv][dim]) per layer."""
    K = np.stack([to_f32(h[layer][0]).reshape(kv, dim) for h in history_kv])   # [T][kv][dim]
    V = np.stack([to_f32(h[layer][1]).reshape(kv, dim) for h in history_kv])
    q = to_f32(q_codes).reshape(qh, dim)
    g = qh // kv
    out = np.zeros((qh, dim), dtype=np.float64)
    for h in range(qh):
        s = K[:, h // g, :].astype(np.float64) @ q[h].astype(np.float64) * scale
        p = np.exp(s - s.max())
        out[h] = (p[:, None] * V[:, h // g, :]).sum(0) / p.sum()
    return out.reshape(-1)


@pytest.mark.parametrize("dim,qh,kv", [(64, 8, 2), (128, 4, 4)])
def test_batched_write_and_attention_many_lanes(host, dev, dim, qh, kv):
    """Ragged lanes decoding through writeLayerBatch + attendLayerBatch with
    engine promotion mid-way; every lane's output is checked against an fp32
    GQA over its own history (tolerance 2e-3 abs + 1e-3 rel)."""
    L, lanes, steps = 2, 6, 80
    rng = np.random.default_rng(dim + qh)
    start = [int(x) for x in rng.integers(1, 40, lanes)]
    engine = host.Engine(L, kv, dim, qh, 1 << 20, 512, 16)
    stream = dev.Stream()
    scale = 1.0 / math.sqrt(dim)
    hist = {r: [] for r in range(lanes)}
    bufs = [Buffers(dev, layers=L, kv=kv, qh=qh, dim=dim, workspace=1 << 20) for _ in range(lanes)]
    for r in range(lanes):
        assert engine.create_request(100 + r) == 0

    def token_kv():
        return [(f16(*rng.uniform(-1, 1, kv * dim)), f16(*rng.uniform(-1, 1, kv * dim))) for _ in range(L)]

    # Prefill each lane token by token through single transactions.
    for r in range(lanes):
        for t in range(start[r]):
            rc, txn = engine.reserve_token(100 + r, t, stream)
            assert rc == 0
            kvs = token_kv()
            q = f16(*rng.uniform(-1, 1, qh * dim))
            dev.copy_to_device(bufs[r].query.ptr, q, stream)
            for layer in range(L):
                dev.copy_to_device(bufs[r].keys[layer].ptr, kvs[layer][0], stream)
                dev.copy_to_device(bufs[r].values[layer].ptr, kvs[layer][1], stream)
                assert txn.write_layer(layer, bufs[r].keys[layer].ptr, bufs[r].values[layer].ptr) == 0
                assert txn.attend_layer(layer, bufs[r].query.ptr, bufs[r].output.ptr, bufs[r].workspace.ptr,
                                        bufs[r].workspace_bytes, scale) == 0
            assert txn.commit() == 0
            hist[r].append(kvs)
    worst = 0.0
    for step in range(steps):
        if step == steps // 2:
            for r in range(lanes):
                rc, _ = engine.promote_request(100 + r, stream)
                assert rc == 0
        txns = []
        for r in range(lanes):
            rc, txn = engine.reserve_token(100 + r, len(hist[r]), stream)
            assert rc == 0
            txns.append(txn)
        kvs = [token_kv() for _ in range(lanes)]
        qs = [f16(*rng.uniform(-1, 1, qh * dim)) for _ in range(lanes)]
        for r in range(lanes):
            dev.copy_to_device(bufs[r].query.ptr, qs[r], stream)
            for layer in range(L):
                dev.copy_to_device(bufs[r].keys[layer].ptr, kvs[r][layer][0], stream)
                dev.copy_to_device(bufs[r].values[layer].ptr, kvs[r][layer][1], stream)
        for layer in range(L):
            st = host.write_layer_batch(txns, [layer] * lanes, [b.keys[layer].ptr for b in bufs],
                                        [b.values[layer].ptr for b in bufs])
            assert st == [0] * lanes
            st = host.attend_layer_batch(
                txns, [(layer, b.query.ptr, b.output.ptr, b.workspace.ptr, b.workspace_bytes, scale) for b in bufs])
            assert st == [0] * lanes
            dev.sync(stream)
            for r in range(lanes):
                got = to_f32(dev.download(bufs[r].output.ptr, (qh * dim,), np.uint16))
                want = _oracle_lane(hist[r] + [kvs[r]], layer, qs[r], qh, kv, dim, scale)
                err = np.abs(got - want)
                assert np.all(err <= 2e-3 + 1e-3 * np.abs(want)), (step, r, layer, err.max())
                worst = max(worst, float(err.max()))
        for r, txn in enumerate(txns):
            assert txn.commit() == 0
            hist[r].append(kvs[r])
    snap = engine.snapshot()
    assert snap.committed_token_count == sum(len(h) for h in hist.values())
    assert snap.batched_write_submissions >= steps * L
    assert snap.allocated_secondary_pages > 0   # promotion published extents
    assert engine.check_invariants()
    for r in range(lanes):
        assert engine.release_request(100 + r) == 0
    stream.destroy()


# --- HipKvCache (tests/cuda/cuda_kv_test.cpp) ------------------------------------------------------------

LAYOUT = (2, 2, 8)


def _append(dev, cache, rid, begin, count, stream):
    data = make_kv_closed_form(*LAYOUT, begin, count)
    buf = dev.upload(data.reshape(-1), stream)
    res = cache.append(rid, count, buf.ptr, stream)
    assert res.ok(), (res.metadata_error, res.device_status)
    return buf


def _gather(dev, cache, rid, count, stream):
    L, H, D = LAYOUT
    out = dev.DeviceBuffer(L * 2 * count * H * D * 2)
    res = cache.gather(rid, out.ptr, stream)
    assert res.ok(), (res.metadata_error, res.device_status)
    return dev.download(out.ptr, (L * 2 * count * H * D,), np.uint16)


def test_cache_append_gather_promotion_attention(host, dev):
    """testAppendGatherPromotionAndAttention, cuda_kv_test.cpp:287-351."""
    L, H, D = LAYOUT
    cache = host.Cache(L, H, D, 16, 2)
    assert cache.status() == 0
    info = cache.storage_info()
    token_bytes = L * 2 * H * D * 2
    assert info.micro_reserved_bytes == 16 * 8 * token_bytes
    assert info.extent_reserved_bytes == 2 * 64 * token_bytes
    stream = dev.Stream()
    assert cache.create_request(1) == 0
    keep = [_append(dev, cache, 1, b, n, stream) for b, n in ((0, 5), (5, 11), (16, 48))]
    expected = make_kv_closed_form(L, H, D, 0, 64).reshape(-1)
    assert np.array_equal(_gather(dev, cache, 1, 64, stream), expected)
    res = cache.promote(1, 0, stream)
    assert res.ok()
    _, entries = cache.block_table(1)
    assert len(entries) == 1 and entries[0][2] == 1
    assert np.array_equal(_gather(dev, cache, 1, 64, stream), expected)

    query = ((np.arange(L * H * D) % 11) + 1).astype(np.float32) * 0.03125
    ref = oracle.reference_attention(L, H, D, expected, 64, query)
    q = dev.upload(query, stream)
    o = dev.DeviceBuffer(query.nbytes)
    assert cache.reference_attention(1, q.ptr, o.ptr, stream).ok()
    got = dev.download(o.ptr, query.shape, np.float32)
    assert np.max(np.abs(got - ref)) <= 5e-4
    assert cache.check_invariants()
    assert cache.release_request(1) == 0
    assert cache.check_invariants()
    del keep
    stream.destroy()


def test_cache_partial_tail_cow(host, dev):
    """testPartialTailCow, cuda_kv_test.cpp:353-391."""
    cache = host.Cache(*LAYOUT, 4, 1)
    stream = dev.Stream()
    assert cache.create_request(10) == 0
    a = _append(dev, cache, 10, 0, 5, stream)
    assert cache.fork_request(10, 11) == 0
    b = _append(dev, cache, 11, 5, 3, stream)
    assert np.array_equal(_gather(dev, cache, 10, 5, stream), make_kv_closed_form(*LAYOUT, 0, 5).reshape(-1))
    assert np.array_equal(_gather(dev, cache, 11, 8, stream), make_kv_closed_form(*LAYOUT, 0, 8).reshape(-1))
    assert cache.check_invariants()
    assert cache.release_request(11) == 0 and cache.release_request(10) == 0
    del a, b
    stream.destroy()


def test_cache_fault_rollback(host, dev):
    """testFaultRollback, cuda_kv_test.cpp:393-454."""
    cache = host.Cache(*LAYOUT, 16, 1)
    stream = dev.Stream()
    assert cache.create_request(20) == 0
    a = _append(dev, cache, 20, 0, 64, stream)
    cache.inject_failure_once("submission")
    res = cache.promote(20, 0, stream)
    assert res.device_status == DEV_SUBMISSION_FAILED
    _, entries = cache.block_table(20)
    assert len(entries) == 8
    snap = cache.snapshot()
    assert snap.promotion_count == 0 and snap.extent_pool.allocated_slots == 0

    cache.inject_failure_once("completion")
    res = cache.promote(20, 0, stream)
    assert res.device_status == DEV_EXECUTION_FAILED
    _, entries = cache.block_table(20)
    assert len(entries) == 8
    assert cache.snapshot().extent_pool.allocated_slots == 0
    assert cache.check_invariants()

    assert cache.create_request(21) == 0
    one = dev.upload(make_kv_closed_form(*LAYOUT, 0, 1).reshape(-1), stream)
    cache.inject_failure_once("submission")
    res = cache.append(21, 1, one.ptr, stream)
    assert res.device_status == DEV_SUBMISSION_FAILED
    assert cache.block_table(21) is None
    assert cache.check_invariants()
    # The surviving request's data is intact and still promotable.
    assert cache.promote(20, 0, stream).ok()
    assert np.array_equal(_gather(dev, cache, 20, 64, stream), make_kv_closed_form(*LAYOUT, 0, 64).reshape(-1))
    assert cache.release_request(20) == 0
    del a
    stream.destroy()


def test_engine_prefill_promotion_then_decode(host, dev):
    """Bulk prefill through the engine (append + seal + promotion), then gather
    is bit-exact against the input and one decode token matches the oracle."""
    L, H, D, QH = 3, 2, 64, 8
    T = 200                                   # 3 extents + one full micro page
    engine = host.Engine(L, H, D, QH, 1 << 16, 64, 8)
    assert engine.permute_free_slots(1, 11) == 0 and engine.permute_free_slots(0, 12) == 0
    assert engine.create_request(5) == 0
    rng = np.random.default_rng(3)
    kv = f16(*rng.uniform(-1, 1, L * 2 * T * H * D)).reshape(L, 2, T, H, D)
    stream = dev.Stream()
    src = dev.upload(kv.reshape(-1), stream)
    rc, promoted = engine.append_prefill(5, T, src.ptr, stream, promote=True)
    assert rc == 0 and promoted == 3
    _, entries = engine.block_table(5)
    assert [e[2] for e in entries] == [1, 1, 1, 0] and entries[-1][1] == 8
    assert engine.snapshot().committed_token_count == T
    assert engine.check_invariants()

    descs = host.descriptors_from_entries(entries)
    d = dev.upload(descs, stream)
    out = dev.DeviceBuffer(kv.nbytes)
    dev.check(dev.lib().kimkv_gather(ctypes.c_void_p(engine.storage_handle()), ctypes.c_void_p(d.ptr), len(descs), T,
                                     ctypes.c_void_p(out.ptr), ctypes.c_void_p(stream.handle)), "gather")
    got = dev.download(out.ptr, kv.shape, np.uint16, stream)
    assert np.array_equal(got, kv)

    buf = Buffers(dev, layers=L, kv=H, qh=QH, dim=D, workspace=1 << 16)
    rc, txn = engine.reserve_token(5, T, stream)
    assert rc == 0
    new = [(f16(*rng.uniform(-1, 1, H * D)), f16(*rng.uniform(-1, 1, H * D))) for _ in range(L)]
    q = f16(*rng.uniform(-1, 1, QH * D))
    dev.copy_to_device(buf.query.ptr, q, stream)
    scale = 1.0 / math.sqrt(D)
    for layer in range(L):
        dev.copy_to_device(buf.keys[layer].ptr, new[layer][0], stream)
        dev.copy_to_device(buf.values[layer].ptr, new[layer][1], stream)
        assert txn.write_layer(layer, buf.keys[layer].ptr, buf.values[layer].ptr) == 0
        assert txn.attend_layer(layer, buf.query.ptr, buf.output.ptr, buf.workspace.ptr, buf.workspace_bytes,
                                scale) == 0
    assert txn.commit() == 0
    hist = [[(kv[l, 0, t].reshape(-1), kv[l, 1, t].reshape(-1)) for l in range(L)] for t in range(T)]
    want = _oracle_lane(hist + [new], L - 1, q, QH, H, D, scale)
    got = to_f32(dev.download(buf.output.ptr, (QH * D,), np.uint16))
    assert np.all(np.abs(got - want) <= 2e-3 + 1e-3 * np.abs(want))
    _, entries = engine.block_table(5)
    assert [e[2] for e in entries] == [1, 1, 1, 0, 0] and entries[-1][1] == 1   # new tail after the sealed page
    assert engine.release_request(5) == 0
    assert engine.check_invariants()
    stream.destroy()


# --- chunked prefill through the engine -------------------------------------------------------------------

def _causal_oracle(K, V, Q, t0, scale, G):
    """fp64 causal GQA: K, V [T][kv][D] f32, Q [n][QH][D] f32; row i attends the first t0 + i + 1 tokens."""
    n = Q.shape[0]
    T = K.shape[0]
    out = np.zeros(Q.shape, dtype=np.float64)
    Kd, Vd, Qd = K.astype(np.float64), V.astype(np.float64), Q.astype(np.float64)
    for h in range(Q.shape[1]):
        s = Qd[:, h, :] @ Kd[:, h // G, :].T * scale                     # [n][T]
        s[np.arange(T)[None, :] > (t0 + np.arange(n))[:, None]] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h, :] = (p @ Vd[:, h // G, :]) / p.sum(axis=1, keepdims=True)
    return out


def test_engine_prefill_chunks_batched(host, dev):
    """Chunks of 37 / 64 / 200 prompt tokens on contexts of 0 / 100 / 1000 tokens
    and on a fork child sharing a partial tail (COW), advanced layer by layer with
    one write launch and one attention launch per layer for all chunks.  Every
    output row matches an fp64 causal GQA (2e-3 abs + 1e-3 rel), the gathered
    KV is bit-exact afterwards and a decode token then matches the oracle."""
    L, H, D, QH = 3, 4, 64, 32
    G = QH // H
    scale = 1.0 / math.sqrt(D)
    engine = host.Engine(L, H, D, QH, 1 << 16, 512, 64)
    assert engine.permute_free_slots(1, 5) == 0 and engine.permute_free_slots(0, 6) == 0
    rng = np.random.default_rng(17)
    stream = dev.Stream()
    contexts = {1: 0, 2: 100, 3: 1000}
    kv = {}
    keep = []
    for rid, t0 in contexts.items():
        assert engine.create_request(rid) == 0
        kv[rid] = f16(*rng.uniform(-1, 1, L * 2 * t0 * H * D)).reshape(L, 2, t0, H, D)
        if t0:
            src = dev.upload(kv[rid].reshape(-1), stream)
            keep.append(src)
            rc, _ = engine.append_prefill(rid, t0, src.ptr, stream, promote=True)
            assert rc == 0, host.ENGINE_ERRORS[rc]
    assert engine.fork_request(2, 4) == 0            # shares request 2's partial micro tail
    kv[4] = kv[2].copy()
    contexts[4] = 100
    chunk_tokens = {1: 37, 2: 64, 3: 200, 4: 45}

    chunks, new_kv, queries, outs = {}, {}, {}, {}
    for rid, n in chunk_tokens.items():
        rc, c = engine.prefill_begin(rid, contexts[rid], n, stream)
        assert rc == 0, host.ENGINE_ERRORS[rc]
        chunks[rid] = c
        new_kv[rid] = f16(*rng.uniform(-1, 1, L * 2 * n * H * D)).reshape(L, 2, n, H, D)
        queries[rid] = f16(*rng.uniform(-1, 1, L * n * QH * D)).reshape(L, n, QH, D)
        outs[rid] = [dev.DeviceBuffer(n * QH * D * 2) for _ in range(L)]
    # An open chunk blocks every other mutation of its request.
    rc, _ = engine.reserve_token(3, 1000 + 200, stream)
    assert host.ENGINE_ERRORS[rc] == "invalid_state"
    assert host.ENGINE_ERRORS[engine.release_request(3)] == "invalid_state"
    assert host.ENGINE_ERRORS[engine.fork_request(3, 9)] == "invalid_state"
    rc, _ = engine.prefill_begin(3, 1000, 8, stream)
    assert host.ENGINE_ERRORS[rc] == "invalid_state"

    order = list(chunk_tokens)
    dkv = {rid: dev.upload(new_kv[rid].reshape(-1), stream) for rid in order}
    dq = {rid: dev.upload(queries[rid].reshape(-1), stream) for rid in order}
    per_layer = {rid: chunk_tokens[rid] * H * D * 2 for rid in order}
    for layer in range(L):
        keys = [dkv[r].ptr + (layer * 2) * per_layer[r] for r in order]
        values = [dkv[r].ptr + (layer * 2 + 1) * per_layer[r] for r in order]
        st = host.prefill_write_batch([chunks[r] for r in order], layer, keys, values)
        assert st == [0] * len(order), st
        qs = [dq[r].ptr + layer * chunk_tokens[r] * QH * D * 2 for r in order]
        st = host.prefill_attend_batch([chunks[r] for r in order], layer, qs, [outs[r][layer].ptr for r in order],
                                       scale)
        assert st == [0] * len(order), st
    for rid in order:
        assert chunks[rid].finish() == 0
        chunks[rid].close()
    assert engine.check_invariants()
    assert engine.snapshot().committed_token_count == sum(contexts[r] + chunk_tokens[r] for r in order)

    worst = 0.0
    for rid in order:
        t0, n = contexts[rid], chunk_tokens[rid]
        full = np.concatenate([kv[rid], new_kv[rid]], axis=2)            # [L][2][T][H][D]
        for layer in range(L):
            want = _causal_oracle(to_f32(full[layer, 0]), to_f32(full[layer, 1]), to_f32(queries[rid][layer]),
                                  t0, scale, G)
            got = to_f32(dev.download(outs[rid][layer].ptr, (n, QH, D), np.uint16))
            err = np.abs(got - want)
            assert np.all(err <= 2e-3 + 1e-3 * np.abs(want)), (rid, layer, float(err.max()))
            worst = max(worst, float(err.max()))
        _, entries = engine.block_table(rid)
        descs = host.descriptors_from_entries(entries)
        d = dev.upload(descs, stream)
        T = t0 + n
        out = dev.DeviceBuffer(full.nbytes)
        dev.check(dev.lib().kimkv_gather(ctypes.c_void_p(engine.storage_handle()), ctypes.c_void_p(d.ptr),
                                         len(descs), T, ctypes.c_void_p(out.ptr), ctypes.c_void_p(stream.handle)),
                  "gather")
        assert np.array_equal(dev.download(out.ptr, full.shape, np.uint16, stream), full), rid
        kv[rid] = full
    print(f"engine prefill chunks max_err={worst:.2e}", flush=True)

    # A decode token after the prompt chunks (request 3, 1200 tokens).
    buf = Buffers(dev, layers=L, kv=H, qh=QH, dim=D, workspace=1 << 16)
    rc, txn = engine.reserve_token(3, 1200, stream)
    assert rc == 0, host.ENGINE_ERRORS[rc]
    new = [(f16(*rng.uniform(-1, 1, H * D)), f16(*rng.uniform(-1, 1, H * D))) for _ in range(L)]
    q = f16(*rng.uniform(-1, 1, QH * D))
    dev.copy_to_device(buf.query.ptr, q, stream)
    for layer in range(L):
        dev.copy_to_device(buf.keys[layer].ptr, new[layer][0], stream)
        dev.copy_to_device(buf.values[layer].ptr, new[layer][1], stream)
        assert txn.write_layer(layer, buf.keys[layer].ptr, buf.values[layer].ptr) == 0
        assert txn.attend_layer(layer, buf.query.ptr, buf.output.ptr, buf.workspace.ptr, buf.workspace_bytes,
                                scale) == 0
    assert txn.commit() == 0
    hist = [[(kv[3][l, 0, t].reshape(-1), kv[3][l, 1, t].reshape(-1)) for l in range(L)] for t in range(1200)]
    want = _oracle_lane(hist + [new], L - 1, q, QH, H, D, scale)
    got = to_f32(dev.download(buf.output.ptr, (QH * D,), np.uint16))
    assert np.all(np.abs(got - want) <= 2e-3 + 1e-3 * np.abs(want))
    for rid in order:
        assert engine.release_request(rid) == 0
    snap = engine.snapshot()
    assert snap.request_count == 0 and snap.allocated_primary_pages == 0 and snap.allocated_secondary_pages == 0
    stream.destroy()


def test_engine_prefill_chunk_errors(host, dev):
    """Layer order, an abandoned chunk and an injected submission failure: the
    last two cancel the request, exactly like a failed bulk append."""
    L, H, D, QH = 2, 2, 64, 4
    engine = host.Engine(L, H, D, QH, 1 << 16, 64, 8)
    stream = dev.Stream()
    n = 20
    k = dev.upload(f16(*np.linspace(-1, 1, n * H * D)), stream)
    q = dev.upload(f16(*np.linspace(1, -1, n * QH * D)), stream)
    o = dev.DeviceBuffer(n * QH * D * 2)
    assert engine.create_request(1) == 0
    rc, c = engine.prefill_begin(1, 5, n, stream)
    assert host.ENGINE_ERRORS[rc] == "invalid_state"          # committed length is 0
    rc, c = engine.prefill_begin(1, 0, n, stream)
    assert rc == 0
    assert host.ENGINE_ERRORS[c.attend_layer(0, q.ptr, o.ptr, 0.125)] == "layer_out_of_order"
    assert host.ENGINE_ERRORS[c.write_layer(1, k.ptr, k.ptr)] == "layer_out_of_order"
    assert c.write_layer(0, k.ptr, k.ptr) == 0
    assert host.ENGINE_ERRORS[c.write_layer(0, k.ptr, k.ptr)] == "layer_out_of_order"
    assert c.attend_layer(0, q.ptr, o.ptr, 0.125) == 0
    assert host.ENGINE_ERRORS[c.finish()] == "invalid_state"  # abandoned after layer 0
    c.close()
    assert host.ENGINE_ERRORS[engine.release_request(1)] == "request_not_found"
    assert engine.snapshot().allocated_primary_pages == 0

    assert engine.create_request(2) == 0
    rc, c = engine.prefill_begin(2, 0, n, stream)
    assert rc == 0
    assert engine.inject_failure_once("submission")
    assert c.write_layer(0, k.ptr, k.ptr) == SUBMISSION_FAILED
    assert c.finish() == SUBMISSION_FAILED
    c.close()
    assert host.ENGINE_ERRORS[engine.release_request(2)] == "request_not_found"

    assert engine.create_request(3) == 0
    rc, c = engine.prefill_begin(3, 0, n, stream)
    assert rc == 0
    for layer in range(L):
        assert c.write_layer(layer, k.ptr, k.ptr) == 0
        assert c.attend_layer(layer, q.ptr, o.ptr, 0.125) == 0
    assert c.finish() == 0
    assert c.finish() == 0                                      # idempotent
    c.close()
    assert engine.snapshot().committed_token_count == n
    assert engine.release_request(3) == 0
    assert engine.check_invariants()
    snap = engine.snapshot()
    assert snap.request_count == 0 and snap.allocated_primary_pages == 0
    stream.destroy()


def _engine_lane_batch_case(host, dev, steps=1, seed=77, groups=1):
    """256 ragged lanes through reserveBatch + writeLayerBatch + attendLayerBatch + commitBatch for
    `steps` tokens: enough (lane, kv head) pairs for the decode planner to take one kv head per workgroup
    with each lane in one chunk (no split-K merge).  Contexts are built by bulk prefill with promotion of
    every full 64-token run; every lane's output at every step is checked against the oracle's fp32 GQA
    decode of its history.  groups > 1 splits the lanes into that many batches, each on its own stream,
    launched one after the other and committed after the next batch's layers are queued (as the
    benchmark pipelines them), so their launches overlap on the GPU."""
    L, H, D, QH, lanes = 2, 4, 64, 32, 256
    HD = H * D
    rng = np.random.default_rng(seed)
    T = [int(t) for t in rng.integers(150, 400, lanes)]
    engine = host.Engine(L, H, D, QH, 1 << 16, sum(t // 8 + 3 + steps for t in T) + 64, sum(t // 64 for t in T) + 16)
    stream = dev.Stream()
    stage = dev.DeviceBuffer(L * 2 * 400 * HD * 2)
    for i in range(lanes):
        assert engine.create_request(i + 1) == 0
        dev.fill_kv(stage.ptr, L, T[i], HD, seed, i, 0, stream)
        rc, _ = engine.append_prefill(i + 1, T[i], stage.ptr, stream, promote=True)
        assert rc == 0
    stream.synchronize()
    newkv = dev.DeviceBuffer(lanes * L * 2 * HD * 2)
    query = dev.DeviceBuffer(lanes * L * QH * D * 2)
    out = dev.DeviceBuffer(lanes * L * QH * D * 2)
    qseed = seed ^ 0x5155
    flags, _, _ = dev.decode_plan(engine.storage_handle(), [t + 1 for t in T], QH)
    assert flags & dev.DECODE_HEAD_SPLIT and (flags & ~dev.DECODE_HEAD_SPLIT) >= max(T) + 1
    # A smaller batch may be planned with split-K chunks: room for their partials.
    ws_lane = max(dev.workspace_bytes(max(T) + steps, 64, QH, D), 256)
    ws = dev.DeviceBuffer(lanes * ws_lane)
    bounds = np.linspace(0, lanes, groups + 1).astype(int)
    streams = [stream] + [dev.Stream() for _ in range(groups - 1)]
    batches = []
    for g in range(groups):
        lane = np.arange(bounds[g], bounds[g + 1], dtype=np.uint64)
        b = host.LaneBatch(engine, lane + np.uint64(1), ws.ptr + lane * np.uint64(ws_lane), ws_lane,
                           1.0 / math.sqrt(D), streams[g])
        for l in range(L):
            b.keys[l, :] = newkv.ptr + np.uint64(2 * HD) * (lane * np.uint64(2 * L) + np.uint64(2 * l))
            b.values[l, :] = newkv.ptr + np.uint64(2 * HD) * (lane * np.uint64(2 * L) + np.uint64(2 * l + 1))
            b.queries[l, :] = query.ptr + np.uint64(2 * QH * D) * (lane * np.uint64(L) + np.uint64(l))
            b.outputs[l, :] = out.ptr + np.uint64(2 * QH * D) * (lane * np.uint64(L) + np.uint64(l))
        batches.append((b, [T[int(i)] for i in lane]))
    worst = 0.0
    for step in range(steps):
        for i in range(lanes):
            t = T[i] + step
            dev.fill_kv(newkv.ptr + i * L * 2 * HD * 2, L, 1, HD, seed, i, t, stream)
            for l in range(L):
                dev.fill_rows(query.ptr + (i * L + l) * QH * D * 2, QH * D, qseed, dev.synth_kv_row(i, l, 0, t),
                              QH * D, stream)
        stream.synchronize()
        pending = None
        for b, Tg in batches:
            b.reserve(np.array([t + step for t in Tg], dtype=np.uint32))
            assert not b.failed()
            for l in range(L):
                b.write(l)
                assert not b.failed(), (l, sorted(set(b.status.tolist())))
                b.attend(l)
                assert not b.failed(), (l, sorted(set(b.status.tolist())))
            if pending is not None:
                pending.commit()
                assert not pending.failed(), sorted(set(pending.status.tolist()))
            pending = b
        pending.commit()
        assert not pending.failed(), sorted(set(pending.status.tolist()))
        dev.sync()
        got = dev.download(out.ptr, (lanes, L, QH * D), np.uint16)
        for i in range(lanes):
            n = T[i] + step + 1
            for l in range(L):
                kv = np.empty((1, 2, n, H, D), dtype=np.uint16)
                for c in range(2):
                    kv[0, c] = oracle.synth_rows(n * HD, seed, oracle.kv_row(i, l, c, 0), HD).reshape(n, H, D)
                pages = (n + 7) // 8
                pools = oracle.HostPools(1, H, D, pages, 1)
                table = np.zeros(pages, dtype=oracle.DESC)
                for k in range(pages):
                    table[k] = (k, 1, 8 * k, min(8, n - 8 * k), 8, 0)
                    pools.append_tokens(kv, n, 8 * k, 0, k, 0, min(8, n - 8 * k))
                q = oracle.synth_rows(QH * D, qseed, oracle.kv_row(i, l, 0, n - 1), QH * D)
                want = pools.paged_decode(table, n, 0, QH, q, 1.0 / math.sqrt(D), f32=True)
                a = got[i, l].view(np.float16).astype(np.float32)
                err = np.abs(a - want)
                assert np.all(err <= 2e-3 + 1e-3 * np.abs(want)), (step, i, l, float(err.max()))
                worst = max(worst, float(err.max()))
    assert engine.check_invariants()
    for extra in streams[1:]:
        extra.destroy()
    print(f"engine lane batch: lanes={lanes} steps={steps} groups={groups} T=[{min(T)},{max(T)}] "
          f"chunk={flags & ~dev.DECODE_HEAD_SPLIT} max_err={worst:.2e}", flush=True)


def test_engine_head_split_batch_matches_oracle(host, dev):
    _engine_lane_batch_case(host, dev)


def test_engine_lane_groups_on_own_streams(host, dev):
    """Two lane batches on two streams whose decode launches overlap (the
    benchmark's default), three tokens each, against the oracle."""
    _engine_lane_batch_case(host, dev, steps=3, seed=78, groups=2)


def test_engine_small_staging_ring(host, dev, monkeypatch):
    """The same lanes with a 64 KiB staging ring (32 KiB per request): the
    first reserve writes every lane's whole device table (~60 KB of patches
    and descriptors, so several patch launches), the later ones patch one
    entry per lane, and the ring wraps with items, jobs and patches
    interleaved, over three steps."""
    monkeypatch.setenv("KIMKV_STAGING_RING_BYTES", str(64 << 10))
    _engine_lane_batch_case(host, dev, steps=3, seed=78)


def _lane_records_run(host, dev, shuffle, steps=3, seed=81, reverse_attend=False, heads=4):
    """24 lanes (two of them forks of one prefix with a partial tail, so their first token copies it on
    write; ragged contexts up to ~3000 tokens, so some lanes split into several chunks) through
    LaneBatch for `steps` tokens.  shuffle: lanes' query and output buffers in a random order (not
    evenly spaced).  reverse_attend: every layer's write and attention take the reserved transactions
    in reverse order (still evenly spaced, with negative strides).  Returns per-step outputs in lane
    order, the engine's lane_record_launches, and the inputs for an oracle check."""
    L, H, D, QH, lanes = 3, heads, 64, 32, 24
    HD, QD = H * D, QH * D
    rng = np.random.default_rng(seed)
    T = [int(t) for t in rng.integers(20, 3000, lanes)]
    P = 1003                                   # the forks' prefix: a partial 8-token tail (1003 % 8 = 3)
    T[-2], T[-1] = P, P
    ws_lane = max(dev.workspace_bytes(max(T) + steps, 64, QH, D), 256)
    engine = host.Engine(L, H, D, QH, ws_lane, sum(t // 8 + 3 + steps for t in T) + 64,
                         sum(t // 64 for t in T) + 16)
    stream = dev.Stream()
    stage = dev.DeviceBuffer(L * 2 * max(T) * HD * 2)
    for i in range(lanes - 2):
        assert engine.create_request(i + 1) == 0
        dev.fill_kv(stage.ptr, L, T[i], HD, seed, i, 0, stream)
        rc, _ = engine.append_prefill(i + 1, T[i], stage.ptr, stream, promote=True)
        assert rc == 0
    root = 1000
    assert engine.create_request(root) == 0
    dev.fill_kv(stage.ptr, L, P, HD, seed, 500, 0, stream)
    assert engine.append_prefill(root, P, stage.ptr, stream, promote=True)[0] == 0
    for i in (lanes - 2, lanes - 1):
        assert engine.fork_request(root, i + 1) == 0
    assert engine.release_request(root) == 0
    stream.synchronize()
    newkv = dev.DeviceBuffer(lanes * L * 2 * HD * 2)
    query = dev.DeviceBuffer(lanes * L * QD * 2)
    out = dev.DeviceBuffer(lanes * L * QD * 2)
    ws = dev.DeviceBuffer(lanes * ws_lane)
    slot = np.random.default_rng(seed + 1).permutation(lanes) if shuffle else np.arange(lanes)
    lane = np.arange(lanes, dtype=np.uint64)
    b = host.LaneBatch(engine, lane + np.uint64(1), ws.ptr + lane * np.uint64(ws_lane), ws_lane, 0.125, stream)
    pos = slot.astype(np.uint64)
    for l in range(L):
        b.keys[l, :] = newkv.ptr + np.uint64(2 * HD) * (lane * np.uint64(2 * L) + np.uint64(2 * l))
        b.values[l, :] = newkv.ptr + np.uint64(2 * HD) * (lane * np.uint64(2 * L) + np.uint64(2 * l + 1))
        b.queries[l, :] = query.ptr + np.uint64(2 * QD) * (np.uint64(l * lanes) + pos)
        b.outputs[l, :] = out.ptr + np.uint64(2 * QD) * (np.uint64(l * lanes) + pos)
    qseed = seed ^ 0x5155
    items = dev.DeviceBuffer(lanes * host.DECODE_ITEM_BYTES)
    outs = []
    for step in range(steps):
        for i in range(lanes):
            t = T[i] + step
            dev.fill_kv(newkv.ptr + i * L * 2 * HD * 2, L, 1, HD, seed, i, t, stream)
            for l in range(L):
                dev.fill_rows(query.ptr + (l * lanes + int(slot[i])) * QD * 2, QD, qseed, dev.synth_kv_row(i, l, 0, t),
                              QD, stream)
        stream.synchronize()
        b.reserve(np.array([t + step for t in T], dtype=np.uint32))
        assert not b.failed()
        for l in range(L):
            if reverse_attend:
                rt = [types.SimpleNamespace(h=int(x)) for x in b.txns[::-1]]
                st = host.write_layer_batch(rt, [l] * lanes, [int(k) for k in b.keys[l, ::-1]],
                                            [int(v) for v in b.values[l, ::-1]])
                assert not any(st), st
                reqs = [(l, int(b.queries[l, i]), int(b.outputs[l, i]), ws.ptr + i * ws_lane, ws_lane, 0.125)
                        for i in reversed(range(lanes))]
                st = host.attend_layer_batch(rt, reqs, items)
                assert not any(st), st
                continue
            b.write(l)
            assert not b.failed(), sorted(set(b.status.tolist()))
            b.attend(l)
            assert not b.failed(), sorted(set(b.status.tolist()))
        b.commit()
        assert not b.failed(), sorted(set(b.status.tolist()))
        dev.sync()
        got = dev.download(out.ptr, (L, lanes, QD), np.uint16)
        outs.append(np.stack([got[:, int(slot[i])] for i in range(lanes)]))   # [lane][layer][QD]
    assert engine.check_invariants()
    launches = engine.lane_record_launches()
    engine.close()
    stream.destroy()
    return outs, launches, T, qseed


def test_engine_lane_records_and_staged_items_agree(host, dev):
    """Batched attention of at most 64 lanes whose queries, outputs, workspaces and new rows are evenly
    spaced launches from device lane records (kimkv_paged_decode_lanes) at every layer: layer 0 copies
    the step's records to the device and the later layers reuse them.  The same lanes with shuffled
    query and output buffers take the staged-item launch at every layer.  The two give the same outputs bit for bit over three token steps of three layers (split-K
    lanes, fresh pages, a fork's copy-on-write tail), and plain lanes match the oracle."""
    even, n_even, T, qseed = _lane_records_run(host, dev, shuffle=False)
    mixed, n_mixed, _, _ = _lane_records_run(host, dev, shuffle=True)
    steps, L = len(even), even[0].shape[1]
    assert n_even == steps * L, n_even
    assert n_mixed == 0, n_mixed
    for s_ in range(steps):
        assert np.array_equal(even[s_], mixed[s_]), s_
    H, D, QH, seed = 4, 64, 32, 81
    HD = H * D
    worst = 0.0
    for i in range(3):                          # plain lanes: the oracle's decode of their history
        n = T[i] + steps
        for l in range(L):
            kv = np.empty((1, 2, n, H, D), dtype=np.uint16)
            for c in range(2):
                kv[0, c] = oracle.synth_rows(n * HD, seed, oracle.kv_row(i, l, c, 0), HD).reshape(n, H, D)
            pages = (n + 7) // 8
            pools = oracle.HostPools(1, H, D, pages, 1)
            table = np.zeros(pages, dtype=oracle.DESC)
            for k in range(pages):
                table[k] = (k, 1, 8 * k, min(8, n - 8 * k), 8, 0)
                pools.append_tokens(kv, n, 8 * k, 0, k, 0, min(8, n - 8 * k))
            q = oracle.synth_rows(QH * D, qseed, oracle.kv_row(i, l, 0, n - 1), QH * D)
            want = pools.paged_decode(table, n, 0, QH, q, 0.125, f32=True)
            a = even[-1][i, l].view(np.float16).astype(np.float32)
            err = np.abs(a - want)
            assert np.all(err <= 2e-3 + 1e-3 * np.abs(want)), (i, l, float(err.max()))
            worst = max(worst, float(err.max()))
    print(f"lane records vs staged items: {steps} steps x {L} layers, record launches {n_even}, "
          f"oracle max err {worst:.2e}", flush=True)


def test_engine_lane_records_in_another_order(host, dev):
    """The reserve call copies the lane records for an attention of its transactions in reservation
    order.  Attending them in reverse order instead (evenly spaced with negative strides) misses that
    copy: layer 0 copies its own records and every layer still launches from records, with the same
    outputs bit for bit as the attention in reservation order."""
    fwd, n_fwd, _, _ = _lane_records_run(host, dev, shuffle=False)
    rev, n_rev, _, _ = _lane_records_run(host, dev, shuffle=False, reverse_attend=True)
    steps, L = len(fwd), fwd[0].shape[1]
    assert n_fwd == steps * L and n_rev == steps * L, (n_fwd, n_rev)
    for s_ in range(steps):
        assert np.array_equal(fwd[s_], rev[s_]), s_


def test_engine_lane_records_eight_kv_heads(host, dev):
    """The lane-record path with 8 kv heads (group 4): two workgroups per chunk share its cached group
    table and the reserve call's records; outputs equal the staged-item launches of shuffled buffers bit
    for bit over three steps, and plain lanes match the oracle."""
    even, n_even, T, qseed = _lane_records_run(host, dev, shuffle=False, heads=8)
    mixed, n_mixed, _, _ = _lane_records_run(host, dev, shuffle=True, heads=8)
    steps, L = len(even), even[0].shape[1]
    assert n_even == steps * L and n_mixed == 0, (n_even, n_mixed)
    for s_ in range(steps):
        assert np.array_equal(even[s_], mixed[s_]), s_
    H, D, QH, seed = 8, 64, 32, 81
    HD = H * D
    for i in range(2):
        n = T[i] + steps
        for l in range(L):
            kv = np.empty((1, 2, n, H, D), dtype=np.uint16)
            for c in range(2):
                kv[0, c] = oracle.synth_rows(n * HD, seed, oracle.kv_row(i, l, c, 0), HD).reshape(n, H, D)
            pages = (n + 7) // 8
            pools = oracle.HostPools(1, H, D, pages, 1)
            table = np.zeros(pages, dtype=oracle.DESC)
            for k in range(pages):
                table[k] = (k, 1, 8 * k, min(8, n - 8 * k), 8, 0)
                pools.append_tokens(kv, n, 8 * k, 0, k, 0, min(8, n - 8 * k))
            q = oracle.synth_rows(QH * D, qseed, oracle.kv_row(i, l, 0, n - 1), QH * D)
            want = pools.paged_decode(table, n, 0, QH, q, 0.125, f32=True)
            a = even[-1][i, l].view(np.float16).astype(np.float32)
            err = np.abs(a - want)
            assert np.all(err <= 2e-3 + 1e-3 * np.abs(want)), (i, l, float(err.max()))


def test_inflight_transaction_pages_survive_sibling_release_and_promotion(host, dev):
    """The engine's token transactions take no page lease (the reference leases every page of the
    candidate table per token, src/cuda/engine/backend.cpp:411-424): a request's committed table holds a
    reference to every page its launches read and the reservation owns the copy-on-write target until
    commit, while the manager refuses release, fork, append and promotion of a request with a live
    reservation.  Checked on the device: a lane batch of two fork children is reserved (each copies the
    shared partial prefix tail) and every layer's write and attention is queued behind a long fill
    kernel on its stream; meanwhile, on another stream, the two sibling forks are released, a third
    request is promoted (its micro pages return to the LIFO free list) and a fourth request allocates
    and writes 4096 tokens of fresh pages.  Had any page of the in-flight lanes been freed, the fourth
    request would have been given it and overwritten it before the decode read it.  The outputs match
    the oracle, the lanes' pages gather bit for bit after commit, and so do the other requests'."""
    L, H, D, QH, seed = 4, 4, 64, 32, 515
    HD, QD = H * D, QH * D
    engine = host.Engine(L, H, D, QH, 1 << 16, 2048, 256)
    assert engine.permute_free_slots(1, seed) == 0 and engine.permute_free_slots(0, seed + 1) == 0
    sa, sb = dev.Stream(), dev.Stream()
    P = 2048 + 3
    stage = dev.DeviceBuffer(L * 2 * 4096 * HD * 2)
    root, kids, promo, fresh = 100, [1, 2, 3, 4], 200, 300
    assert engine.create_request(root) == 0
    dev.fill_kv(stage.ptr, L, P, HD, seed, 7, 0, sa)
    rc, _ = engine.append_prefill(root, P, stage.ptr, sa, promote=True)
    assert rc == 0
    for k in kids:
        assert engine.fork_request(root, k) == 0
    assert engine.release_request(root) == 0
    assert engine.create_request(promo) == 0
    dev.fill_kv(stage.ptr, L, 512, HD, seed, 8, 0, sa)
    rc, promoted = engine.append_prefill(promo, 512, stage.ptr, sa, promote=False)
    assert rc == 0 and promoted == 0
    sa.synchronize()
    tables_before = {k: engine.block_table(k)[1] for k in kids[:2]}

    lanes = np.arange(2, dtype=np.uint64)
    newkv = dev.DeviceBuffer(2 * L * 2 * HD * 2)
    query = dev.DeviceBuffer(2 * L * QD * 2)
    out = dev.DeviceBuffer(2 * L * QD * 2)
    qseed = seed ^ 0x77
    for i in range(2):
        dev.fill_kv(newkv.ptr + i * L * 2 * HD * 2, L, 1, HD, seed, 50 + i, P, sa)
        for l in range(L):
            dev.fill_rows(query.ptr + (i * L + l) * QD * 2, QD, qseed, dev.synth_kv_row(i, l, 0, P), QD, sa)
    ws_lane = max(dev.workspace_bytes(P + 1, 64, QH, D), 256)          # room for any split-K plan
    ws = dev.DeviceBuffer(2 * ws_lane)
    b = host.LaneBatch(engine, lanes + np.uint64(1), ws.ptr + lanes * np.uint64(ws_lane), ws_lane, 0.125, sa)
    for l in range(L):
        b.keys[l, :] = newkv.ptr + np.uint64(2 * HD) * (lanes * np.uint64(2 * L) + np.uint64(2 * l))
        b.values[l, :] = newkv.ptr + np.uint64(2 * HD) * (lanes * np.uint64(2 * L) + np.uint64(2 * l + 1))
        b.queries[l, :] = query.ptr + np.uint64(2 * QD) * (lanes * np.uint64(L) + np.uint64(l))
        b.outputs[l, :] = out.ptr + np.uint64(2 * QD) * (lanes * np.uint64(L) + np.uint64(l))
    delay = dev.DeviceBuffer(1 << 31)
    sa.synchronize()
    for rep in range(2):                                               # ~4 GB of stores ahead of the lanes
        dev.fill_rows(delay.ptr, 1 << 30, rep, 0, 1 << 16, sa)
    b.reserve(np.array([P, P], dtype=np.uint32))
    assert not b.failed()
    for l in range(L):
        b.write(l)
        b.attend(l)
    assert not b.failed(), sorted(set(b.status.tolist()))
    # While the lanes' launches wait behind the fill: the in-flight requests are pinned ...
    conflict = host.ENGINE_ERRORS.index("request_conflict")
    assert engine.release_request(1) == conflict
    assert engine.fork_request(1, 999) == conflict
    # ... and their siblings, a promotion and fresh allocations go ahead on another stream.
    assert engine.release_request(3) == 0 and engine.release_request(4) == 0
    rc, promoted = engine.promote_request(promo, sb)
    assert rc == 0 and promoted == 8
    assert engine.create_request(fresh) == 0
    fresh_stage = dev.DeviceBuffer(L * 2 * 4096 * HD * 2)
    dev.fill_kv(fresh_stage.ptr, L, 4096, HD, seed, 9, 0, sb)
    rc, _ = engine.append_prefill(fresh, 4096, fresh_stage.ptr, sb, promote=True)
    assert rc == 0
    sb.synchronize()
    b.commit()
    assert not b.failed(), sorted(set(b.status.tolist()))
    assert engine.check_invariants()
    got = dev.download(out.ptr, (2, L, QD), np.uint16)
    T = P + 1
    for i, k in enumerate(kids[:2]):
        hist = np.empty((L, 2, T, H, D), dtype=np.uint16)
        for l in range(L):
            for c in range(2):
                hist[l, c, :P] = oracle.synth_rows(P * HD, seed, oracle.kv_row(7, l, c, 0), HD).reshape(P, H, D)
                hist[l, c, P] = oracle.synth_rows(HD, seed, oracle.kv_row(50 + i, l, c, P), HD).reshape(H, D)
        for l in range(L):
            q = oracle.synth_rows(QD, qseed, oracle.kv_row(i, l, 0, P), QD)
            pools = oracle.HostPools(1, H, D, (T + 7) // 8, 1)
            table = np.zeros((T + 7) // 8, dtype=oracle.DESC)
            for g in range(len(table)):
                n = min(8, T - 8 * g)
                table[g] = (g, 1, 8 * g, n, 8, 0)
                pools.append_tokens(hist[l:l + 1], T, 8 * g, 0, g, 0, n)
            want = pools.paged_decode(table, T, 0, QH, q, 0.125, f32=True)
            a = to_f32(got[i, l])
            assert np.all(np.abs(a - want) <= 2e-3 + 1e-3 * np.abs(want)), (k, l)
        _, entries = engine.block_table(k)
        assert entries[:-1] == tables_before[k][:-1] and entries[-1][1] == 4      # COW tail: 3 copied + 1
        assert entries[-1][3] != tables_before[k][-1][3]
        descs = host.descriptors_from_entries(entries)
        d = dev.upload(descs)
        buf = dev.DeviceBuffer(hist.nbytes)
        dev.check(dev.lib().kimkv_gather(ctypes.c_void_p(engine.storage_handle()), ctypes.c_void_p(d.ptr),
                                         len(descs), T, ctypes.c_void_p(buf.ptr), None), "gather")
        assert np.array_equal(dev.download(buf.ptr, hist.shape, np.uint16), hist), k
    for rid, sid, n in ((promo, 8, 512), (fresh, 9, 4096)):
        _, entries = engine.block_table(rid)
        descs = host.descriptors_from_entries(entries)
        d = dev.upload(descs)
        buf = dev.DeviceBuffer(L * 2 * n * HD * 2)
        dev.check(dev.lib().kimkv_gather(ctypes.c_void_p(engine.storage_handle()), ctypes.c_void_p(d.ptr),
                                         len(descs), n, ctypes.c_void_p(buf.ptr), None), "gather")
        want = np.empty((L, 2, n, H, D), dtype=np.uint16)
        for l in range(L):
            for c in range(2):
                want[l, c] = oracle.synth_rows(n * HD, seed, oracle.kv_row(sid, l, c, 0), HD).reshape(n, H, D)
        assert np.array_equal(dev.download(buf.ptr, want.shape, np.uint16), want), rid
    del delay
    sa.destroy()
    sb.destroy()
