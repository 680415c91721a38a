"""Test configuration: `gpu` marks tests that need an MI355X (gfx950).

CPU tests (-m "not gpu") pin the oracle against the reference's golden
vectors and check host logic; GPU tests compare the HIP kernels, called
through the C ABI, with the oracle.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def zo():
    from oracle import zo as _zo
    _zo.load()
    return _zo


@pytest.fixture(scope="session")
def ctx():
    import zero_amd
    c = zero_amd.Context(int(os.environ.get("ZG_DEVICE", "0")))
    yield c
    c.close()
