"""The reference's own CPU contract tests, compiled from its sources against
this build's headers and linked with its libkimkv.so (oracle/build.py,
build_reference_contracts): page pool, block table / COW / fork, page
leases, promotion, the engine SPI transaction contract, the generation
runtime, the iteration scheduler, the binary16 codec + reference attention
and the weight manifest.  Each binary must exit 0.  Skipped where the reference tree (and
so the binaries) is absent."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "oracle", "_ref", "contracts")
NAMES = ["page_pool_test", "block_table_test", "page_lease_test", "promotion_test", "engine_kv_contract_test",
         "generation_runtime_test", "iteration_scheduler_test", "kv_reference_test", "weight_manifest_test"]


@pytest.mark.parametrize("name", NAMES)
def test_reference_contract(name):
    path = os.path.join(BIN, name)
    if not os.path.exists(path):
        if os.path.isdir(os.environ.get("KIMKV_REFERENCE_TREE", "/root/reference")):
            pytest.fail(f"{path} is missing: run __graft_entry__.build() first")
        pytest.skip("the reference tree is not present here")
    proc = subprocess.run([path], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout
