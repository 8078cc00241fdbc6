import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libasca_hip.so")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (test infrastructure), built on first use."""
    from oracle import pyoracle

    pyoracle.lib()
    return pyoracle


@pytest.fixture(scope="session")
def g():
    """The Gpu handle.  On a GPU run a missing device or library is a failure,
    never a skip: the HIP path must be the one that runs."""
    from asca_amd import gpu

    dev = gpu.gpu()
    if dev is None:
        pytest.fail(f"no usable GPU backend: {gpu.describe()}")
    return dev
