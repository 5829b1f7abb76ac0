import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "ops-sparse_amd"), os.path.join(REPO, "oracle"), REPO):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def pytest_sessionstart(session):
    """Builds the HIP library once if nothing is built yet (hipcc cross-compiles without a GPU)."""
    from ops_sparse import _lib

    if not os.path.exists(_lib.LIB_PATH):
        from ops_sparse.build import build_library

        build_library()
