import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP plugin)")


@pytest.fixture(scope="session")
def plugin():
    # PyTorch-ROCm ships its own HIP runtime.  Loading it before the plugin makes the
    # plugin bind to that runtime, so tests that mix torch tensors and plugin calls in
    # one process see one HIP runtime (bench.py imports torch first for the same reason).
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    import webgpu_amd
    return webgpu_amd.Plugin()


@pytest.fixture(scope="session")
def ctx(plugin):
    if plugin.device_count() < 1:
        pytest.skip("no HIP device")
    c = plugin.create_context(0)
    yield c
    c.close()
