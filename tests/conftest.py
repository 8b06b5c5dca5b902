"""Test configuration: import paths and markers.

Mirrors /root/reference/tests/conftest.py:9-23 (source path + markers), with
``gpu`` marking every test that launches the HIP kernels on a ROCm device.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "kda-ascendc_amd", ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running case")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _no_fused_wait_gave_up(request):
    """After every GPU test: no fused-kernel work-group gave up a bounded
    wait (kda_bt16_fused_aborts; such a work-group writes NaN instead of
    hanging the GPU, and the count is how a caller can tell)."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    import torch

    if not torch.cuda.is_available():
        return
    from kda_bt16 import fused_abort_count

    n = fused_abort_count(reset=True)
    assert n == 0, f"{n} fused-kernel work-groups gave up a wait during {request.node.nodeid}"
