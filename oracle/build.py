"""Build recipe for the CPU oracle (TEST INFRASTRUCTURE ONLY).

  oracle/libkvoracle.so        gcc build of kvoracle.c (the C restatement)
  oracle/_ref/libkimkv_ref.so  g++ build of the reference's own CPU sources
                               (src/core, src/runtime, src/reference, read in
                               place under the reference tree) plus
                               oracle/ref_driver.cpp; only when that tree exists.
  oracle/_ref/contracts/*      the reference's own CPU contract tests (its
                               tests/core, tests/runtime, tests/engine and
                               tests/reference sources, read in place) compiled
                               against THIS build's include/ and linked with its
                               libkimkv.so: the reference's checks run against
                               the drop-in (build_reference_contracts, after the
                               package is built).
All outputs are git-ignored and stay off GPU runs (nothing there uses them).
"""
from __future__ import annotations

import glob
import os
import subprocess

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(ORACLE_DIR)
REFERENCE = os.environ.get("KIMKV_REFERENCE_TREE", "/root/reference")


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed: {' '.join(cmd)}\n{proc.stdout}")


def build_oracle() -> str:
    out = os.path.join(ORACLE_DIR, "libkvoracle.so")
    # IEEE float semantics: no contraction, no fast-math.
    _run(["gcc", "-std=c11", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-Wall",
          os.path.join(ORACLE_DIR, "kvoracle.c"), "-o", out + ".tmp", "-lm"])
    os.replace(out + ".tmp", out)
    return out


def reference_sources() -> list[str]:
    srcs = []
    for sub in ("src/core", "src/runtime", "src/reference"):
        srcs += sorted(glob.glob(os.path.join(REFERENCE, sub, "*.cpp")))
    return srcs


def build_reference() -> str | None:
    srcs = reference_sources()
    if not srcs or not os.path.isdir(os.path.join(REFERENCE, "include")):
        return None
    out_dir = os.path.join(ORACLE_DIR, "_ref")
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, "libkimkv_ref.so")
    _run(["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-pthread",
          f"-I{os.path.join(REFERENCE, 'include')}", f"-I{os.path.join(REPO, 'include')}",
          *srcs, os.path.join(ORACLE_DIR, "ref_driver.cpp"), "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


# Reference tests whose includes this build provides (the fixed-size page
# strategy is not part of it).
REFERENCE_CONTRACTS = (
    "core/page_pool_test",
    "runtime/block_table_test",
    "runtime/page_lease_test",
    "runtime/promotion_test",
    "engine/engine_kv_contract_test",
    "engine/generation_runtime_test",
    "engine/iteration_scheduler_test",
    "reference/kv_reference_test",
    "model/weight_manifest_test",
)


def build_reference_contracts() -> list[str]:
    """Compiles the reference's contract tests against include/ and libkimkv.so."""
    lib_dir = os.path.join(REPO, "kim-kvcache_amd", "_lib")
    srcs = [os.path.join(REFERENCE, "tests", t + ".cpp") for t in REFERENCE_CONTRACTS]
    if not all(os.path.exists(s) for s in srcs) or not os.path.exists(os.path.join(lib_dir, "libkimkv.so")):
        return []
    out_dir = os.path.join(ORACLE_DIR, "_ref", "contracts")
    os.makedirs(out_dir, exist_ok=True)
    outs = []
    for src in srcs:
        out = os.path.join(out_dir, os.path.splitext(os.path.basename(src))[0])
        _run(["g++", "-std=c++17", "-O1", f"-I{os.path.join(REPO, 'include')}", src, f"-L{lib_dir}", "-lkimkv",
              "-lkimkv_hip", f"-Wl,-rpath,{lib_dir}", "-pthread", "-o", out + ".tmp"])
        os.replace(out + ".tmp", out)
        outs.append(out)
    return outs


def build_all() -> list[str]:
    built = [build_oracle()]
    ref = build_reference()
    if ref:
        built.append(ref)
    return built


if __name__ == "__main__":
    for p in build_all():
        print(p)
