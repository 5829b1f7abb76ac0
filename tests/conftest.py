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
    """Builds the HIP library if it is missing or was built from other sources (hipcc
    cross-compiles without a GPU); the loader refuses a stale library."""
    from ops_sparse import _lib
    from ops_sparse.build import build_library, file_build_id, source_hash

    # read from the file, not dlopen'ed: a library loaded once stays mapped
    # under its path for the life of the process
    if file_build_id(_lib.LIB_PATH) != source_hash():
        build_library()
