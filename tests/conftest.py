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


# Launch policies of the kernel families: "valu" the VALU kernels (the row-block kernels at
# one row, the general GEMV for 2-8), "general" the general VALU GEMV at every row count,
# "mfma" the matrix-core kernels for every row count, "default" the library's defaults.
PATHS = {
    "valu": dict(mfma_rows_q4=0, mfma_rows_q8=0),
    "general": dict(mfma_rows_q4=0, mfma_rows_q8=0, rowblock=0),
    "mfma": dict(mfma_rows_q4=1, mfma_rows_q8=1),
    "default": {},
}


def _scope(path: str):
    from llmnputest_amd import ops
    return ops.policy_scope(ops.Policy(**PATHS[path]))


@pytest.fixture(params=["valu", "general", "mfma"])
def kpath(request, dev):
    """Run the test once on each kernel family."""
    with _scope(request.param):
        yield request.param


@pytest.fixture(params=["valu", "general"])
def vpath(request, dev):
    """Run the test on each VALU kernel family (row-block at one row, and the general one)."""
    with _scope(request.param):
        yield request.param


@pytest.fixture
def valu(dev):
    """Pin the VALU kernels (row-block at one row)."""
    with _scope("valu"):
        yield


@pytest.fixture
def general(dev):
    """Pin the general VALU GEMV (for tests of its own splits)."""
    with _scope("general"):
        yield


@pytest.fixture
def mfma(dev):
    """Pin the matrix-core kernels for every row count."""
    with _scope("mfma"):
        yield


@pytest.fixture(params=["mfma", "valu"])
def apath(request, dev):
    """Run an attention test on each attention kernel (matrix-core and VALU)."""
    from llmnputest_amd import ops
    with ops.policy_scope(ops.Policy(attn_mfma=int(request.param == "mfma"))):
        yield request.param
