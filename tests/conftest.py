import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs the HIP kernels")


@pytest.fixture(scope="session")
def cuda_device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _no_gave_up_waits(request):
    """GPU tests: no bounded in-kernel wait (the batched GEMM's LDS counter) may give up.
    Such a wait ends after ~1 ms so that every kernel exits; had one ended that way, the
    results could be wrong although they matched, so the test fails."""
    if request.node.get_closest_marker("gpu") is None:
        yield
        return
    import torch

    if not torch.cuda.is_available():
        yield
        return
    from moeinfra_amd import _lib

    torch.cuda.synchronize()
    _lib.wait_timeouts(reset=True)
    yield
    torch.cuda.synchronize()
    assert _lib.wait_timeouts(reset=True) == 0, "a bounded in-kernel wait gave up"
