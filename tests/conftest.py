import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    # The native library must load on a GPU box: a missing build is a failure,
    # not a skip.
    from orthossm_amd import _native
    _native.load()
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _no_lookback_fault(request):
    """After every GPU test: no workspace the test used reports a look-back
    wait that gave up (the header's fault word, read through
    osm_workspace_status)."""
    yield
    if request.node.get_closest_marker("gpu") is None or not gpu_available():
        return
    from orthossm_amd import ops
    bad = ops.workspace_faults(reset=True)
    assert not bad, f"look-back fault word set after {request.node.nodeid}: {bad}"
