import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def reference():
    """The reference's own CPU kernels (oracle/_ref), where they were built."""
    import oracle as oracle_pkg

    if not oracle_pkg.has_reference():
        pytest.skip("oracle/_ref/libmfref.so is not built (the reference sources are absent)")
    return oracle_pkg.Reference()


@pytest.fixture(scope="session")
def stream():
    """A stream on rocm:0. A GPU test fails (not skips) when there is no gfx950 device."""
    import mensurflow_amd as mf

    count = mf.device_count()
    assert count > 0, "no gfx950 device visible: GPU tests need an MI355X"
    s = mf.Stream(0)
    yield s
    s.close()
