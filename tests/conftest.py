import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "stockfish-trainer_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

LIB = os.path.join(PKG, "lib", "libsft_ft.so")
ORACLE_LIB = os.path.join(ROOT, "oracle", "_build", "libft_oracle.so")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (runs the HIP kernels)")


def _have_gpu() -> bool:
    try:
        import torch

        return torch.cuda.is_available() and torch.cuda.device_count() > 0
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if any("gpu" in item.keywords for item in items) and not _have_gpu():
        skip = pytest.mark.skip(reason="no GPU visible")
        for item in items:
            if "gpu" in item.keywords:
                item.add_marker(skip)


@pytest.fixture(scope="session", autouse=True)
def _built():
    """Build the library and the oracle only when nothing is built yet."""
    if not os.path.exists(LIB) or not os.path.exists(ORACLE_LIB):
        import __graft_entry__

        __graft_entry__.build()
    yield


def golden(name: str):
    import numpy as np

    return np.load(os.path.join(ROOT, "tests", "golden", name + ".npz"), allow_pickle=False)
