import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "gemma4-rs_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def ctx():
    """The backend context on cuda:0; the HIP library must be built and a GPU present."""
    import torch
    import g4hip

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a GPU: run with -m 'not gpu' on the CPU")
    torch.cuda.init()
    c = g4hip.Context(0)
    yield c
    c.close()
