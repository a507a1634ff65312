import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def coracle():
    """The C restatement, built on first use (it ships prebuilt to the GPU box)."""
    from oracle import oracle

    if not os.path.exists(oracle.LIB):
        oracle.build()
    return oracle
