import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The GPU tests' device.  Missing GPU or library is a failure, never a skip:
    these tests only run where the HIP path must be the one that runs."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu-marked test without a visible GPU")
    from leanstack_amd import _lib

    _lib.load()
    name = torch.cuda.get_device_name(0)
    print(f"[gpu] {name}; library {_lib.LIBRARY_PATH}", flush=True)
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before any GPU work so that a crashed run still says which.
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[case] {request.node.nodeid}", flush=True)
        sys.stdout.flush()
    yield
    if request.node.get_closest_marker("gpu") is not None and os.environ.get("LSK_SYNC_EACH_TEST", "1") == "1":
        import torch

        if torch.cuda.is_available():
            torch.cuda.synchronize()
