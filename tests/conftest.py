"""Test configuration: the `gpu` marker and import paths.

`-m "not gpu"` runs the oracle checks against the golden fixtures, the host
logic of the C ABI and the library's symbol exports (no GPU needed);
`-m gpu` runs the parity tests of the HIP path against the oracle.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "sera.c_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a visible MI355X (HIP) device")


@pytest.fixture(scope="session")
def golden_dir():
    return os.path.join(ROOT, "tests", "golden")
