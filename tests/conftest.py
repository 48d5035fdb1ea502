import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


def golden(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def _gpu_available():
    try:
        import qraf_amd  # noqa: F401  (raises if libqraf_hip.so is missing)
        from qraf_amd.backend import device_count
    except ImportError:
        return None  # library not built: GPU tests must fail, not skip
    return device_count() > 0


@pytest.fixture(scope="session")
def hip():
    """The HIP backend, initialised on device 0.  GPU tests fail loudly if the
    library is missing and skip only when no device is visible."""
    avail = _gpu_available()
    if avail is None:
        pytest.fail("qraf_amd/libqraf_hip.so is not built or failed to load")
    if not avail:
        pytest.skip("no GPU visible")
    import qraf_amd
    qraf_amd.backend.backend_init(0)
    return qraf_amd


@pytest.fixture(scope="session")
def reference():
    """The compiled reference (oracle/_ref/libqraf_ref.so).  GPU parity tests
    that need it fail, not skip, when it is missing: it is built by
    `make -C oracle all` where the reference checkout exists and travels with
    the working tree."""
    from oracle import pyoracle as po
    if po.ref() is None:
        pytest.fail("oracle/_ref/libqraf_ref.so (the compiled reference) is missing; build it with `make -C oracle all`")
    return po.ref()
