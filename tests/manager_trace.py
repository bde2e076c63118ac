"""Trace harness for KvCacheManager parity.

`ManagerLib(cdll, prefix)` binds the kimkv_manager_* facade of libkimkv.so
(prefix "kimkv_") or the same functions of the compiled reference in
oracle/_ref (prefix "kvref_").  `random_trace` produces a seeded operation
sequence; `run_trace` executes it and records every return code, id, table,
page record and pool snapshot, so two implementations can be compared
record for record.
"""
from __future__ import annotations

import ctypes
import random

U32, U64 = ctypes.c_uint32, ctypes.c_uint64


class Entry(ctypes.Structure):
    _fields_ = [("logical_token_begin", U32), ("valid_tokens", ctypes.c_uint16), ("kind", ctypes.c_uint8),
                ("reserved", ctypes.c_uint8), ("slot", U32), ("generation", U32)]


class Handle(ctypes.Structure):
    _fields_ = [("kind", U32), ("slot", U32), ("generation", U32)]


class PageMeta(ctypes.Structure):
    _fields_ = [("state", U32), ("valid_tokens", U32), ("ref_count", U32), ("promotion_pins", U32),
                ("inflight_readers", U32), ("reserved", U32), ("mutable_owner", U64)]


class PoolSnap(ctypes.Structure):
    _fields_ = [("kind", U32), ("total_slots", U32), ("free_slots", U32), ("allocated_slots", U32),
                ("successful_allocations", U64), ("successful_releases", U64), ("failed_allocations", U64),
                ("rejected_releases", U64)]


class MgrSnap(ctypes.Structure):
    _fields_ = [("request_count", U64), ("promotion_count", U64), ("page_lease_count", U64),
                ("token_reservation_count", U64), ("micro_pool", PoolSnap), ("extent_pool", PoolSnap)]


def _pool_tuple(p):
    return (p.kind, p.total_slots, p.free_slots, p.allocated_slots, p.successful_allocations,
            p.successful_releases, p.failed_allocations, p.rejected_releases)


class ManagerLib:
    def __init__(self, cdll: ctypes.CDLL, prefix: str):
        self.lib = cdll
        self.p = prefix
        f = self._fn
        f("manager_create", ctypes.c_void_p, [U32, U32])
        f("manager_destroy", None, [ctypes.c_void_p])
        for name in ["create_request", "seal_tail", "release_request"]:
            f("manager_" + name, ctypes.c_int, [ctypes.c_void_p, U64])
        f("manager_append", ctypes.c_int, [ctypes.c_void_p, U64, U32])
        f("manager_reserve_token", ctypes.c_int, [ctypes.c_void_p, U64, U32, ctypes.POINTER(U64),
                                                  ctypes.POINTER(U64), ctypes.c_void_p, U32, ctypes.POINTER(U32)])
        for name in ["commit_token", "rollback_token", "commit_promotion", "rollback_promotion", "release_lease"]:
            f("manager_" + name, ctypes.c_int, [ctypes.c_void_p, U64])
        f("manager_fork_request", ctypes.c_int, [ctypes.c_void_p, U64, U64])
        f("manager_prepare_promotion", ctypes.c_int, [ctypes.c_void_p, U64, U32, ctypes.POINTER(U64),
                                                      ctypes.c_void_p, ctypes.c_void_p])
        for name in ["acquire_request_lease", "acquire_promotion_lease", "acquire_reservation_lease"]:
            f("manager_" + name, ctypes.c_int, [ctypes.c_void_p, U64, ctypes.POINTER(U64)])
        f("manager_block_table", ctypes.c_int, [ctypes.c_void_p, U64, ctypes.POINTER(U64), ctypes.c_void_p, U32,
                                                ctypes.POINTER(U32)])
        f("manager_page_metadata", ctypes.c_int, [ctypes.c_void_p, Handle, ctypes.POINTER(PageMeta)])
        f("manager_get_snapshot", None, [ctypes.c_void_p, ctypes.POINTER(MgrSnap)])
        f("manager_check_invariants", ctypes.c_int, [ctypes.c_void_p])
        f("manager_permute_free_slots", ctypes.c_int, [ctypes.c_void_p, U32, U64])
        f("seeded_permutation", None, [U64, U32, ctypes.c_void_p])

    def _fn(self, name, restype, argtypes):
        fn = getattr(self.lib, self.p + name)
        fn.restype = restype
        fn.argtypes = argtypes
        setattr(self, name, fn)


class Manager:
    def __init__(self, ml: ManagerLib, micro: int, extent: int):
        self.ml = ml
        self.h = ml.manager_create(micro, extent)
        assert self.h, "manager_create failed"

    def close(self):
        if self.h:
            self.ml.manager_destroy(self.h)
            self.h = None

    def table(self, rid):
        version, count = U64(), U32()
        rc = self.ml.manager_block_table(self.h, rid, ctypes.byref(version), None, 0, ctypes.byref(count))
        if rc != 0:
            return None
        buf = (Entry * max(count.value, 1))()
        rc = self.ml.manager_block_table(self.h, rid, ctypes.byref(version), buf, count.value, ctypes.byref(count))
        assert rc == 0
        return (version.value, [(e.logical_token_begin, e.valid_tokens, e.kind, e.slot, e.generation)
                                for e in buf[:count.value]])

    def page(self, kind, slot, gen):
        m = PageMeta()
        if self.ml.manager_page_metadata(self.h, Handle(kind, slot, gen), ctypes.byref(m)) != 0:
            return None
        return (m.state, m.valid_tokens, m.ref_count, m.promotion_pins, m.inflight_readers, m.mutable_owner)

    def snapshot(self):
        s = MgrSnap()
        self.ml.manager_get_snapshot(self.h, ctypes.byref(s))
        return (s.request_count, s.promotion_count, s.page_lease_count, s.token_reservation_count,
                _pool_tuple(s.micro_pool), _pool_tuple(s.extent_pool))

    def invariants(self):
        return self.ml.manager_check_invariants(self.h)

    def op(self, name, *args):
        """Runs one operation; returns (code, outputs...)."""
        m = self.ml
        h = self.h
        if name == "create":
            return (m.manager_create_request(h, args[0]),)
        if name == "append":
            return (m.manager_append(h, args[0], args[1]),)
        if name == "reserve":
            rid, version, count = U64(), U64(), U32()
            buf = (Entry * 4096)()
            rc = m.manager_reserve_token(h, args[0], args[1], ctypes.byref(rid), ctypes.byref(version), buf, 4096,
                                         ctypes.byref(count))
            table = [(e.logical_token_begin, e.valid_tokens, e.kind, e.slot, e.generation) for e in buf[:count.value]]
            return (rc, rid.value, version.value if rc == 0 else 0, table if rc == 0 else [])
        if name in ("commit_token", "rollback_token", "commit_promotion", "rollback_promotion", "release_lease",
                    "seal", "release"):
            fn = {"seal": m.manager_seal_tail, "release": m.manager_release_request}.get(name)
            fn = fn or getattr(m, "manager_" + name)
            return (fn(h, args[0]),)
        if name == "fork":
            return (m.manager_fork_request(h, args[0], args[1]),)
        if name == "prepare":
            pid = U64()
            src = (Handle * 8)()
            tgt = Handle()
            rc = m.manager_prepare_promotion(h, args[0], args[1], ctypes.byref(pid), src, ctypes.byref(tgt))
            return (rc, pid.value, [(s.kind, s.slot, s.generation) for s in src] if rc == 0 else [],
                    (tgt.kind, tgt.slot, tgt.generation) if rc == 0 else None)
        if name in ("lease_request", "lease_promotion", "lease_reservation"):
            fn = {"lease_request": m.manager_acquire_request_lease,
                  "lease_promotion": m.manager_acquire_promotion_lease,
                  "lease_reservation": m.manager_acquire_reservation_lease}[name]
            lid = U64()
            rc = fn(h, args[0], ctypes.byref(lid))
            return (rc, lid.value)
        if name == "permute":
            return (m.manager_permute_free_slots(h, args[0], args[1]),)
        if name == "invariants":
            return (self.invariants(),)
        raise ValueError(name)

    def state(self, request_ids):
        """Everything observable: tables of all known ids, their pages, snapshot."""
        tables = {rid: self.table(rid) for rid in sorted(request_ids)}
        pages = {}
        for t in tables.values():
            if t is None:
                continue
            for (_b, _v, kind, slot, gen) in t[1]:
                pages[(kind, slot, gen)] = self.page(kind, slot, gen)
        return tables, pages, self.snapshot()


def random_trace(seed: int, length: int, micro: int, extent: int):
    """A seeded op list.  Arguments that depend on state (reservation,
    promotion and lease ids, promotion begins) are symbolic and resolved at
    run time from the implementation under test, identically for both."""
    rng = random.Random(seed)
    ops = []
    for _ in range(length):
        r = rng.random()
        rid = rng.randint(1, 6)
        if r < 0.07:
            ops.append(("create", rid))
        elif r < 0.30:
            ops.append(("append", rid, rng.choice([1, 1, 2, 3, 5, 7, 8, 9, 15, 16, 17, 31, 64, 64, 70, 130])))
        elif r < 0.45:
            ops.append(("reserve_cycle", rid, rng.choice(["commit", "commit", "commit", "rollback", "hold"])))
        elif r < 0.50:
            ops.append(("seal", rid))
        elif r < 0.58:
            ops.append(("fork", rid, rng.randint(1, 9)))
        elif r < 0.63:
            ops.append(("release", rid))
        elif r < 0.78:
            ops.append(("promote_cycle", rid, rng.randint(0, 40), rng.choice(["commit", "commit", "rollback", "hold"])))
        elif r < 0.86:
            ops.append(("lease", rid))
        elif r < 0.92:
            ops.append(("release_oldest_lease",))
        elif r < 0.96:
            ops.append(("finish_held",))
        else:
            ops.append(("invariants",))
    return ops


def run_trace(mgr: Manager, ops, check_state_every: int = 1):
    """Executes a trace; returns the list of records."""
    records = []
    held_reservations = []   # (rid, reservation id)
    held_promotions = []
    leases = []
    known = set(range(1, 10))
    for i, op in enumerate(ops):
        kind = op[0]
        if kind == "reserve_cycle":
            rid, finish = op[1], op[2]
            t = mgr.table(rid)
            expected = sum(e[1] for e in t[1]) if t else 0
            res = mgr.op("reserve", rid, expected)
            rec = [("reserve", rid, expected, res)]
            if res[0] == 0:
                lease = mgr.op("lease_reservation", res[1])
                rec.append(("lease_reservation", lease))
                if lease[0] == 0:
                    leases.append(lease[1])
                if finish == "hold":
                    held_reservations.append(res[1])
                else:
                    rec.append((finish, mgr.op(finish + "_token", res[1])))
            records.append(tuple(rec))
        elif kind == "promote_cycle":
            rid, pick, finish = op[1], op[2], op[3]
            t = mgr.table(rid)
            begin = pick
            if t and t[1]:
                e = t[1]
                runs = [i for i in range(len(e) - 7) if all(x[2] == 0 and x[1] == 8 for x in e[i:i + 8])]
                # Mostly start at an 8-page micro run (eligible unless shared or
                # pinned), sometimes at an arbitrary entry (not eligible).
                if runs and pick % 4 != 0:
                    begin = e[runs[pick % len(runs)]][0]
                else:
                    begin = e[pick % len(e)][0]
            res = mgr.op("prepare", rid, begin)
            rec = [("prepare", rid, begin, res)]
            if res[0] == 0:
                lease = mgr.op("lease_promotion", res[1])
                rec.append(("lease_promotion", lease))
                if finish == "hold":
                    held_promotions.append((res[1], lease[1] if lease[0] == 0 else 0))
                else:
                    if lease[0] == 0:
                        rec.append(("release_lease", mgr.op("release_lease", lease[1])))
                    rec.append((finish, mgr.op(finish + "_promotion", res[1])))
            records.append(tuple(rec))
        elif kind == "lease":
            res = mgr.op("lease_request", op[1])
            if res[0] == 0:
                leases.append(res[1])
            records.append(("lease", op[1], res))
        elif kind == "release_oldest_lease":
            if leases:
                lid = leases.pop(0)
                records.append(("release_lease", lid, mgr.op("release_lease", lid)))
            else:
                records.append(("release_lease", None))
        elif kind == "finish_held":
            rec = []
            while held_reservations:
                r = held_reservations.pop(0)
                rec.append(("commit_token", r, mgr.op("commit_token", r)))
            while held_promotions:
                pid, lid = held_promotions.pop(0)
                if lid:
                    rec.append(("release_lease", lid, mgr.op("release_lease", lid)))
                rec.append(("commit_promotion", pid, mgr.op("commit_promotion", pid)))
            records.append(tuple(rec))
        elif kind == "fork":
            records.append(("fork", op[1], op[2], mgr.op("fork", op[1], op[2])))
        elif kind == "invariants":
            records.append(("invariants", mgr.op("invariants")))
        else:
            records.append((kind, op[1:], mgr.op(kind, *op[1:])))
        if check_state_every and i % check_state_every == 0:
            records.append(("state", mgr.state(known)))
    # Drain everything so release paths with Retiring pages are exercised.
    rec = []
    for r in held_reservations:
        rec.append(("rollback_token", r, mgr.op("rollback_token", r)))
    for pid, lid in held_promotions:
        rec.append(("rollback_promotion", pid, mgr.op("rollback_promotion", pid)))
        if lid:
            rec.append(("release_lease", lid, mgr.op("release_lease", lid)))
    for lid in leases:
        rec.append(("release_lease", lid, mgr.op("release_lease", lid)))
    for rid in sorted(known):
        rec.append(("release", rid, mgr.op("release", rid)))
    rec.append(("invariants", mgr.op("invariants")))
    records.append(tuple(rec))
    records.append(("final", mgr.state(known)))
    return records
