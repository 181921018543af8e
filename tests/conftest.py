import os
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libmyelin_hip.so")


def _gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session", autouse=True)
def _oracle_built():
    from oracle import c_ref
    from tests.hip import build as test_kernels

    c_ref.build()
    # the test-only HIP kernels (tests/hip/*.hip) are built here when absent,
    # so a fresh checkout needs only `python -m myelin_amd.build`
    if not test_kernels.LIB.exists():
        test_kernels.build()
    yield
