"""Test configuration: paths, the `gpu` marker, shared fixtures.

CPU tests (``-m "not gpu"``) check the oracle against independent pins, the
C ABI's host logic and the workload generators.  GPU tests (``-m gpu``) run
the gfx950 kernels through the C ABI and compare them with the oracle.
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "triton-ext_amd"), os.path.join(REPO, "oracle"), os.path.join(REPO, "tests"), REPO):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long CPU sweep, opt-in via TX_SLOW=1")


def _have_gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    markexpr = (config.getoption("-m") or "").strip()
    strict = markexpr == "gpu"
    have = None
    for item in items:
        if "slow" in item.keywords and os.environ.get("TX_SLOW") != "1":
            item.add_marker(pytest.mark.skip(reason="slow sweep: set TX_SLOW=1"))
        if "gpu" in item.keywords:
            if have is None:
                have = _have_gpu()
            # With `-m gpu` the tests run and the `dev` fixture fails loudly.
            if not have and not strict:
                item.add_marker(pytest.mark.skip(reason="no GPU visible"))


@pytest.fixture(scope="session")
def oracle():
    import oracle as O
    O.build()
    return O


@pytest.fixture(scope="session")
def tx():
    import tx as T
    return T


@pytest.fixture(scope="session")
def dev(tx):
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU tests selected but no GPU is visible")
    d = torch.device("cuda:0")
    tx.init()
    return d
