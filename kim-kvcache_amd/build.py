"""Build recipe for the kim-kv MI355X libraries (in-tree, no cmake).

Outputs (git-ignored, shipped with the tree):
  kim-kvcache_amd/_lib/libkimkv_hip.so  -- gfx950 kernels + the C-ABI of include/kimkv_hip.h
  kim-kvcache_amd/_lib/libkimkv.so      -- C++ host layer (page pool, block tables,
                                           KvCacheManager, token transactions, HIP engine
                                           backend, generation runtime, iteration scheduler)
                                           + the C facade of include/kimkv_host.h
  kim-kvcache_amd/_lib/tests/*          -- C++ contract tests (tests/cpp), run by pytest
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_DIR)
LIB_DIR = os.path.join(PKG_DIR, "_lib")
OBJ_DIR = os.path.join(PKG_DIR, "_lib", "obj")
HIP_SRC = os.path.join(PKG_DIR, "csrc", "hip")
HOST_SRC = os.path.join(PKG_DIR, "csrc", "host")
INCLUDE = os.path.join(REPO, "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ARCH = "gfx950"

# Packed FP32 VALU forms are kept out of every HIP object.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
HOST_FLAGS = ["-std=c++17", "-O2", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        sys.stderr.write(out + "\n")


def _sources(directory: str, suffixes: tuple[str, ...]) -> list[str]:
    found = []
    for root, _dirs, files in os.walk(directory):
        for name in sorted(files):
            if name.endswith(suffixes):
                found.append(os.path.join(root, name))
    return sorted(found)


def _obj_name(src: str, tag: str) -> str:
    rel = os.path.relpath(src, PKG_DIR).replace(os.sep, "_")
    return os.path.join(OBJ_DIR, f"{tag}_{os.path.splitext(rel)[0]}.o")


def _parallel(jobs: list[list[str]]) -> None:
    workers = max(1, min(8, os.cpu_count() or 1))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        for fut in [pool.submit(_run, j) for j in jobs]:
            fut.result()


def build_device() -> str:
    """Compile the HIP kernels into libkimkv_hip.so."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = _sources(HIP_SRC, (".hip",))
    objs = [_obj_name(s, "hip") for s in srcs]
    _parallel([[HIPCC, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{HIP_SRC}", "-c", s, "-o", o]
               for s, o in zip(srcs, objs)])
    out = os.path.join(LIB_DIR, "libkimkv_hip.so")
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-lhipblaslt", "-o", tmp])
    os.replace(tmp, out)
    return out


def build_host() -> str | None:
    """Compile the C++ host layer into libkimkv.so (links libkimkv_hip.so)."""
    srcs = _sources(HOST_SRC, (".cpp",))
    if not srcs:
        return None
    os.makedirs(OBJ_DIR, exist_ok=True)
    objs = [_obj_name(s, "host") for s in srcs]
    _parallel([[CXX, *HOST_FLAGS, f"-I{INCLUDE}", f"-I{HOST_SRC}", "-c", s, "-o", o]
               for s, o in zip(srcs, objs)])
    out = os.path.join(LIB_DIR, "libkimkv.so")
    tmp = out + ".tmp"
    _run([CXX, "-shared", "-fPIC", *objs, f"-L{LIB_DIR}", "-lkimkv_hip",
          "-Wl,-rpath,$ORIGIN", "-pthread", "-o", tmp])
    os.replace(tmp, out)
    return out


TEST_SRC = os.path.join(REPO, "tests", "cpp")
TEST_BIN = os.path.join(LIB_DIR, "tests")


def build_tests() -> list[str]:
    """Compile the C++ contract tests (tests/cpp/*.cpp) against libkimkv.so."""
    srcs = _sources(TEST_SRC, (".cpp",)) if os.path.isdir(TEST_SRC) else []
    os.makedirs(TEST_BIN, exist_ok=True)
    outs = [os.path.join(TEST_BIN, os.path.splitext(os.path.basename(s))[0]) for s in srcs]
    _parallel([[CXX, *HOST_FLAGS, f"-I{INCLUDE}", f"-I{HOST_SRC}", s, f"-L{LIB_DIR}", "-lkimkv", "-lkimkv_hip",
                "-Wl,-rpath,$ORIGIN/..", "-pthread", "-o", o] for s, o in zip(srcs, outs)])
    return outs


def build_all() -> list[str]:
    if os.path.isdir(OBJ_DIR):
        shutil.rmtree(OBJ_DIR)
    built = [build_device()]
    host = build_host()
    if host:
        built.append(host)
        built.extend(build_tests())
    shutil.rmtree(OBJ_DIR, ignore_errors=True)
    return built


if __name__ == "__main__":
    for path in build_all():
        print(path)
