import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "furiosa-opt_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library on cuda:0)")
    config.addinivalue_line("markers", "slow: minutes of CPU work; runs only with FO_SLOW=1 in the environment")


def pytest_collection_modifyitems(config, items):
    if os.environ.get("FO_SLOW") == "1":
        return
    skip = pytest.mark.skip(reason="slow (minutes of oracle work); set FO_SLOW=1 to run")
    for item in items:
        if "slow" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def rt():
    import furiosa_hip as fh

    r = fh.Runtime(int(os.environ.get("FO_HIP_DEVICE", "0")))
    yield r
    r.close()


@pytest.fixture(scope="session")
def rt_eager():
    """A second runtime created with FO_EAGER=1: it defers nothing (zero fills run at allocation,
    casts, map chains and broadcasts when issued), the reference the deferred forms are held to."""
    import furiosa_hip as fh

    old = os.environ.get("FO_EAGER")
    os.environ["FO_EAGER"] = "1"
    try:
        r = fh.Runtime(int(os.environ.get("FO_HIP_DEVICE", "0")))
    finally:
        if old is None:
            del os.environ["FO_EAGER"]
        else:
            os.environ["FO_EAGER"] = old
    yield r
    r.close()
