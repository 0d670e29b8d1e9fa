import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


def pytest_sessionstart(session):
    # A fresh checkout holds no built library (it is kept out of history): build
    # it once, as __graft_entry__.build() would, when nothing is built yet.
    from checkers_amd import build as b
    if not os.path.exists(b.LIB):
        b.build(verbose=False)


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import checkers_amd as ck
    ck.lib()  # loud failure if the library is missing
    return torch.device("cuda:0")
