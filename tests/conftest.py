import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs on the MI355X box)")


def pytest_collection_modifyitems(config, items):
    # Order: CPU tests first, then GPU tests in file order; names starting test_zz_ stay last.
    pass


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as O

    O.lib()
    return O


@pytest.fixture(scope="session")
def ref_lib():
    from oracle import oracle as O

    R = O.ref()
    if R is None:
        pytest.skip("reference CPU objects (oracle/_ref) not built here")
    return R


@pytest.fixture(scope="session")
def gpu():
    from rapidllm_amd import hip

    hip.require_gpu()
    return hip
