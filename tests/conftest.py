import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")
    config.addinivalue_line("markers", "timing: asserts measured cycle ratios; always collected last")


def pytest_collection_modifyitems(session, config, items):
    """Tests that assert timing ratios run after every other test (stable
    order otherwise): a timing outlier on some box must not stop a -x run
    before the parity tests."""
    items[:] = ([it for it in items if it.get_closest_marker("timing") is None] +
                [it for it in items if it.get_closest_marker("timing") is not None])


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def oracle():
    from oracle import race_oracle
    race_oracle._lib()
    return race_oracle


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm device")
    return torch.device("cuda:0")
