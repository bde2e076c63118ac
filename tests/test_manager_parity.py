"""KvCacheManager parity: libkimkv.so vs the reference's own CPU library.

Page tables must be bit-exact: every return code, reservation / promotion /
lease id, block table (version, begin, valid, kind, slot, generation), page
record and pool counter is compared after each operation of seeded traces.
The reference side is oracle/_ref (built from the reference sources) when
present, and always the committed fixtures in tests/golden/manager_traces.json
that the same library produced.
"""
import ctypes
import json
import os

import pytest

import oracle
from tests.golden.make_manager_traces import CASES, _norm
from tests.manager_trace import Manager, ManagerLib, random_trace, run_trace

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "manager_traces.json")


@pytest.fixture(scope="module")
def ours(kimkv):
    path = os.path.join(os.path.dirname(kimkv.device.LIB_PATH), "libkimkv.so")
    return ManagerLib(ctypes.CDLL(path), "kimkv_")


def _run(ml, seed, length, micro, extent, every=3):
    m = Manager(ml, micro, extent)
    try:
        return _norm(run_trace(m, random_trace(seed, length, micro, extent), check_state_every=every))
    finally:
        m.close()


def test_golden_traces(ours):
    cases = json.load(open(GOLDEN))
    assert len(cases) == len(CASES)
    for case in cases:
        got = _run(ours, case["seed"], case["length"], case["micro"], case["extent"])
        assert len(got) == len(case["records"])
        for i, (a, b) in enumerate(zip(got, case["records"])):
            assert a == b, f"seed {case['seed']} record {i}: {a} != {b}"


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (reference tree absent)")
@pytest.mark.parametrize("seed", range(100, 140))
def test_random_traces_match_reference(ours, seed):
    ref = ManagerLib(oracle.ref(), "kvref_")
    micro = [8, 16, 24, 40, 64][seed % 5]
    extent = [1, 3, 6, 12][seed % 4]
    a = _run(ours, seed, 150, micro, extent, every=1)
    b = _run(ref, seed, 150, micro, extent, every=1)
    for i, (x, y) in enumerate(zip(a, b)):
        assert x == y, f"record {i}: ours {x} != reference {y}"
    assert len(a) == len(b)


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (reference tree absent)")
@pytest.mark.parametrize("kind,n", [(0, 1), (0, 37), (1, 5), (1, 64)])
def test_permute_free_slots_matches_reference(ours, kind, n):
    ref = ManagerLib(oracle.ref(), "kvref_")
    results = []
    for ml in (ours, ref):
        m = Manager(ml, 64 if kind == 1 else n, n if kind == 1 else 4)
        assert m.op("permute", kind, 99)[0] == 0
        m.op("create", 1)
        recs = []
        for _ in range(min(n, 8)):
            if kind == 0:
                recs.append(m.op("append", 1, 8))
            else:
                recs.append(m.op("append", 1, 64))
                t = m.table(1)
                recs.append(m.op("prepare", 1, t[1][-8][0]))
                recs.append(m.op("commit_promotion", recs[-1][1]))
        recs.append(m.table(1))
        recs.append(m.snapshot())
        assert m.invariants() == 1
        m.close()
        results.append(_norm(recs))
    assert results[0] == results[1]


def test_permutation_matches_helper(ours):
    from tests.helpers import splitmix_permutation
    out = (ctypes.c_uint32 * 1000)()
    ours.seeded_permutation(12345, 1000, out)
    assert list(out) == list(splitmix_permutation(12345, 1000))


# ---- known answers from the reference's contract tests -------------------------------

def _mgr(ours, micro, extent):
    return Manager(ours, micro, extent)


def test_append_and_lookup_known_answers(ours):
    # tests/runtime/block_table_test.cpp:35-164
    m = _mgr(ours, 8, 2)
    assert m.op("create", 1) == (0,)
    assert m.op("append", 1, 3) == (0,)
    v, entries = m.table(1)
    assert v == 1 and entries == [(0, 3, 0, 0, 1)]
    assert m.page(0, 0, 1)[:3] == (1, 3, 1) and m.page(0, 0, 1)[5] == 1     # Mutable, owner 1
    assert m.op("append", 1, 5) == (0,)
    assert m.table(1)[1] == [(0, 8, 0, 0, 1)]
    assert m.page(0, 0, 1)[0] == 2 and m.page(0, 0, 1)[5] == 0              # Sealed, no owner
    assert m.op("append", 1, 9) == (0,)
    v, entries = m.table(1)
    assert v == 3 and [(e[0], e[1]) for e in entries] == [(0, 8), (8, 8), (16, 1)]
    assert m.invariants() == 1
    assert m.op("release", 1) == (0,)
    snap = m.snapshot()
    assert snap[0] == 0 and snap[4][2] == snap[4][1]                         # all micro pages free
    m.close()


def test_partial_fork_copy_on_write_known_answers(ours):
    # tests/runtime/block_table_test.cpp:166-327
    m = _mgr(ours, 4, 1)
    m.op("create", 10)
    m.op("append", 10, 3)
    before = m.table(10)
    assert m.op("fork", 10, 11) == (0,)
    child = m.table(11)
    assert child[0] == 1 and child[1] == before[1]                           # child version 1, shared page
    assert m.table(10)[0] == before[0]                                       # fork does not bump the source
    h = before[1][0]
    assert m.page(h[2], h[3], h[4])[:3] == (2, 3, 2)                         # sealed, ref 2
    assert m.op("append", 11, 1) == (0,)                                     # COW into a new micro page
    child = m.table(11)
    assert child[1][0][3] != h[3] and child[1][0][1] == 4
    assert m.page(h[2], h[3], h[4])[2] == 1
    assert m.invariants() == 1
    m.close()


def test_full_page_fork_shares_without_copy(ours):
    # tests/runtime/block_table_test.cpp:329-400
    m = _mgr(ours, 4, 1)
    m.op("create", 1)
    m.op("append", 1, 8)
    m.op("fork", 1, 2)
    assert m.op("append", 2, 1) == (0,)
    t1, t2 = m.table(1)[1], m.table(2)[1]
    assert t2[0] == t1[0] and len(t2) == 2                                   # full page shared, new tail
    m.close()


def test_cow_out_of_memory_rolls_back(ours):
    # tests/runtime/block_table_test.cpp:402-468
    m = _mgr(ours, 1, 1)
    m.op("create", 1)
    m.op("append", 1, 3)
    m.op("fork", 1, 2)
    before = m.table(2)
    snap = m.snapshot()
    assert m.op("append", 2, 1) == (5,)                                      # ResourceExhausted
    assert m.table(2) == before
    assert m.snapshot()[4][2] == snap[4][2]
    assert m.invariants() == 1
    m.close()


def test_reservation_commit_and_rollback(ours):
    # tests/runtime/token_reservation_test.cpp:21-150
    m = _mgr(ours, 4, 1)
    m.op("create", 1)
    m.op("append", 1, 7)
    rc, rid, version, table = m.op("reserve", 1, 7)
    assert rc == 0 and rid == 1 and version == 2 and table[-1][1] == 8
    assert m.op("reserve", 1, 7)[0] == 4                                     # RequestConflict
    assert m.op("append", 1, 1) == (4,)
    assert m.op("commit_token", rid) == (0,)
    assert m.table(1)[1][-1][1] == 8
    rc, rid2, _, table = m.op("reserve", 1, 8)                               # tail full -> new micro page
    assert rc == 0 and len(table) == 2
    assert m.op("rollback_token", rid2) == (0,)
    assert len(m.table(1)[1]) == 1
    assert m.op("reserve", 1, 5)[0] == 6                                     # InvalidState: wrong position
    assert m.invariants() == 1
    m.close()


def test_promotion_known_answers(ours):
    # tests/runtime/promotion_test.cpp
    m = _mgr(ours, 16, 2)
    m.op("create", 1)
    m.op("append", 1, 70)
    rc, pid, sources, target = m.op("prepare", 1, 0)
    assert rc == 0 and len(sources) == 8 and target[0] == 1
    assert m.op("prepare", 1, 0)[0] == 8                                     # PromotionNotEligible (pinned)
    assert m.op("reserve", 1, 70)[0] == 4                                    # RequestConflict while promoting
    assert m.op("commit_promotion", pid) == (0,)
    v, entries = m.table(1)
    assert entries[0] == (0, 64, 1, target[1], target[2]) and len(entries) == 2
    assert m.op("commit_promotion", pid) == (9,)                              # PromotionNotFound
    rc, pid2, _, _ = m.op("prepare", 1, 64)
    assert rc == 8
    assert m.invariants() == 1
    m.close()
