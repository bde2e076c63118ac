import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from _loader import load_package  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def kimkv():
    return load_package()


@pytest.fixture(scope="session")
def dev(kimkv):
    d = kimkv.device
    if d.device_count() == 0:
        pytest.fail("no HIP device visible: GPU tests need the MI355X")
    return d
