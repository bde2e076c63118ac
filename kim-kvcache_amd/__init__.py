"""kim-kv for MI355X: host-side Python mirror of the reference's paged-KV API.

The directory name is not a Python identifier, so callers load it with
`load_package()` from `_loader.py` (tests, bench.py and __graft_entry__.py do),
which registers it as the module `kim_kvcache_amd`.

Submodules:
  device  -- ctypes binding of include/kimkv_hip.h (gfx950 kernels, libkimkv_hip.so)
  host    -- ctypes binding of include/kimkv_host.h (C++ host layer, libkimkv.so)
"""
from . import device  # noqa: F401

__all__ = ["device"]
