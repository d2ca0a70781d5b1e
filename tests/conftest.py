import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    import torch
    from llmnputest_amd import _lib
    _lib.lib()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")


def _set_kernel_path(path: str) -> None:
    """Which kernels the GEMV / fused entry points use: the VALU GEMV only, the matrix-core
    kernels for every row count, or the library's default policy."""
    from llmnputest_amd import ops
    q4, q8 = {"valu": (0, 0), "mfma": (1, 1), "default": (2, 1)}[path]
    ops.set_mfma_rows("q4", q4)
    ops.set_mfma_rows("q8", q8)


@pytest.fixture(params=["valu", "mfma"])
def kpath(request, dev):
    """Run the test once on each kernel family."""
    _set_kernel_path(request.param)
    yield request.param
    _set_kernel_path("default")


@pytest.fixture
def valu(dev):
    """Pin the VALU GEMV (for tests of its own knobs)."""
    _set_kernel_path("valu")
    yield
    _set_kernel_path("default")


@pytest.fixture
def mfma(dev):
    """Pin the matrix-core kernels for every row count."""
    _set_kernel_path("mfma")
    yield
    _set_kernel_path("default")


@pytest.fixture(params=["mfma", "valu"])
def apath(request, dev):
    """Run an attention test on each attention kernel (matrix-core and VALU)."""
    from llmnputest_amd import ops
    ops.set_attn_mfma(request.param == "mfma")
    yield request.param
    ops.set_attn_mfma(True)
