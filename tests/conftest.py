import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")
    config.addinivalue_line("markers", "slow: long-running CPU check")


@pytest.fixture(scope="session")
def oracle():
    from oracle import pyoracle

    pyoracle.lib()
    return pyoracle


@pytest.fixture(scope="session")
def ref(oracle):
    if not oracle.ref_available():
        pytest.skip("reference kernels/cpu build (oracle/_ref) not present")
    return oracle.ref_lib()


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import polykernel_amd
    from polykernel_amd import _lib

    _lib.load()  # fails loudly when the HIP library is missing
    return torch.device("cuda:0")
