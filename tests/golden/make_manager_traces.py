"""Writes tests/golden/manager_traces.json: seeded KvCacheManager operation
traces executed by the reference's own CPU library (oracle/_ref, compiled
from the reference sources by oracle/build.py) with every observable result
recorded.  Run from the repository root after __graft_entry__.build():

    python tests/golden/make_manager_traces.py
"""
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from tests.manager_trace import Manager, ManagerLib, random_trace, run_trace  # noqa: E402

CASES = [  # (seed, length, micro pages, extent pages)
    (1, 120, 24, 4), (2, 120, 48, 6), (3, 200, 16, 2), (4, 160, 64, 8), (5, 90, 12, 2), (6, 200, 40, 12),
    (7, 300, 96, 16),
]


def normalize(obj):
    return json.loads(json.dumps(obj, default=lambda o: list(o) if isinstance(o, tuple) else str(o),
                                 sort_keys=True), object_hook=None) if False else _norm(obj)


def _norm(obj):
    if isinstance(obj, dict):
        return {str(k): _norm(v) for k, v in sorted(obj.items(), key=lambda kv: str(kv[0]))}
    if isinstance(obj, (list, tuple)):
        return [_norm(v) for v in obj]
    return obj


def main():
    ml = ManagerLib(oracle.ref(), "kvref_")
    out = []
    for seed, length, micro, extent in CASES:
        ops = random_trace(seed, length, micro, extent)
        m = Manager(ml, micro, extent)
        records = run_trace(m, ops, check_state_every=3)
        m.close()
        out.append({"seed": seed, "length": length, "micro": micro, "extent": extent,
                    "ops": _norm(ops), "records": _norm(records)})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "manager_traces.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
