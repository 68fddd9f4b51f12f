import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "fast-arm-tbcnn_amd" / "python"))
sys.path.insert(0, str(ROOT / "fast-arm-tbcnn_amd" / "lib"))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libtbn_hip.so)")


@pytest.fixture(scope="session")
def orc():
    import oracle_api
    return oracle_api


@pytest.fixture(scope="session")
def tbn():
    """The C++ runtime's Python module (fast-arm-tbcnn_amd/lib/_tbn*.so)."""
    import _tbn
    return _tbn


@pytest.fixture(scope="session")
def dev():
    """The HIP device for GPU tests; fails (never skips) when it is absent."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible HIP device"
    import tbn_hip
    tbn_hip.call("tbn_hip_device_check")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _release_device_buffers():
    yield
    mod = sys.modules.get("gpu_util")
    if mod is not None:
        mod.release()
