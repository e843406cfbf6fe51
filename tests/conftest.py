"""Shared fixtures.  GPU tests carry @pytest.mark.gpu; everything else runs on CPU."""
import os
import shutil
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__ as graft  # noqa: E402

_PKG = os.path.join(ROOT, "fbgemm-ascend_amd")
_BUILT = all(os.path.exists(os.path.join(_PKG, f)) for f in ("libtbe_hip.so", "_tbe_torch.so"))
if not _BUILT and shutil.which("hipcc"):
    graft.build()  # a fresh checkout on the CPU side: compile before collecting tests


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs under `-m gpu`)")


@pytest.fixture(scope="session")
def pkg():
    return graft.load_package()


@pytest.fixture(scope="session")
def oracle():
    return graft.load_oracle()


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    return np.load(os.path.join(ROOT, "tests", "golden", "library_vectors.npz"), allow_pickle=False)


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
