import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def gx():
    import gfxinfer_amd
    gfxinfer_amd.lib()
    return gfxinfer_amd


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import gfxinfer_amd
    gfxinfer_amd.check(gfxinfer_amd.lib().gfxinfer_require_gfx950_device(0))
    return torch.device("cuda:0")


def golden(name: str):
    return np.load(os.path.join(TESTS, "golden", name), allow_pickle=False)
