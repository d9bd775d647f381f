import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libprism_kv.so")


@pytest.fixture(scope="session")
def gpu():
    """The ROCm device for GPU tests; fails (not skips) when absent, so a GPU run cannot pass
    silently without the native path."""
    import torch

    from prism_amd import _lib

    assert torch.cuda.is_available(), "gpu-marked test needs a ROCm device"
    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    return dev


@pytest.fixture(autouse=True)
def _gpu_status_clean(request):
    """Every GPU test must leave the device status word clear (no bad page ids seen)."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    import torch

    if not torch.cuda.is_available():
        return
    from prism_amd.attention import _status, read_status

    for idx in list(_status):
        # the device word and whatever a poll_status has moved to the host meanwhile
        v = read_status(torch.device("cuda", idx), clear=True)
        assert v == 0, f"kernel status flags set: {v}"
