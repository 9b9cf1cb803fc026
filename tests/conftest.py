import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X); runs the HIP kernels")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.lib()
    return o


@pytest.fixture(scope="session")
def lib():
    from metal_linalg_amd import _lib

    return _lib


@pytest.fixture(scope="session")
def api():
    from metal_linalg_amd import api as a

    return a


@pytest.fixture(scope="session")
def cuda():
    """torch with a GPU; GPU tests fail loudly without one (no fallback)."""
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from metal_linalg_amd import _lib

    arch = _lib.hip_arch().decode()
    print(f"[gpu] device={_lib.device_name().decode()} arch={arch} cus={_lib.gpu_core_count()}", flush=True)
    return torch
