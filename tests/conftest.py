import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI library)")


@pytest.fixture(scope="session")
def pkg():
    """The product package (directory `qwen3-vl-jax_amd/`, imported as `qwen3_vl_jax_amd`)."""
    from __graft_entry__ import load_package
    return load_package()


@pytest.fixture(scope="session")
def lib(pkg):
    """The loaded HIP C-ABI library (raises if it was not built)."""
    return pkg.capi.load()


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(autouse=True)
def _skip_gpu_without_device(request):
    if request.node.get_closest_marker("gpu") is not None and not gpu_available():
        pytest.skip("needs a GPU")
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
