"""Registers the kim-kvcache_amd directory as the importable package `kim_kvcache_amd`."""
import importlib.util
import os
import sys

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "kim-kvcache_amd")


def load_package():
    if "kim_kvcache_amd" in sys.modules:
        return sys.modules["kim_kvcache_amd"]
    spec = importlib.util.spec_from_file_location(
        "kim_kvcache_amd", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    module = importlib.util.module_from_spec(spec)
    sys.modules["kim_kvcache_amd"] = module
    spec.loader.exec_module(module)
    return module
