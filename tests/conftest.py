import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long CPU-side test")


@pytest.fixture
def exact_libm():
    """Run the oracle's transcendentals correctly rounded, as the HIP kernels
    compute them, for the tests that require the device bit-exact; the
    oracle's default is glibc's expf/logf/sinf/cosf, what the reference's
    Rust f32 calls use."""
    import zg_oracle as O
    with O.libm_mode(O.LIBM_CORRECT):
        yield
