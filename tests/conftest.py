import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)


GOLDEN = ROOT / "tests" / "golden"


def _load(name):
    import numpy as np

    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def golden_c0():
    return _load("c0_reconstruct.npz")


@pytest.fixture(scope="session")
def golden_anchored():
    return _load("anchored_reconstruct.npz")


@pytest.fixture(scope="session")
def golden_torsion():
    return _load("torsion_small.npz")
