import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs the HIP kernels")


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    return np.load(ROOT / "tests" / "golden" / "golden_attn.npz")


@pytest.fixture(scope="session")
def golden_kv():
    import numpy as np

    return np.load(ROOT / "tests" / "golden" / "golden_kv.npz")


@pytest.fixture(scope="session")
def hip():
    """The native library on a real GPU (gpu tests only).  No fallback: fails loudly."""
    import torch

    from nexus_amd import capi

    if not torch.cuda.is_available():
        pytest.fail("gpu test collected on a host without a HIP device")
    capi.load()
    return capi
