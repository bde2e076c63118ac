"""Runs the C++ tests built from tests/cpp (CPU only).  generation_contract_test
uses a fake KV backend and a fake model and mirrors the reference's
tests/engine scenarios for the single-request generation runtime and the
iteration scheduler; staging_ring_test replays allocation sequences through
the staging ring's region bookkeeping; manager_delta_test runs the
manager's delta append and reservation paths against its reference-form calls
on twin managers."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "kim-kvcache_amd", "_lib", "tests")


@pytest.mark.parametrize("name", ["generation_contract_test", "staging_ring_test", "kv_reference_test", "sha256_test",
                                  "manager_delta_test"])
def test_cpp_contract(name):
    path = os.path.join(BIN, name)
    if not os.path.exists(path):
        pytest.fail(f"{path} is missing: run __graft_entry__.build() first")
    proc = subprocess.run([path], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout
