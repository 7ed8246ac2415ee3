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


@pytest.fixture(scope="session")
def rt():
    import furiosa_hip as fh

    r = fh.Runtime(int(os.environ.get("FO_HIP_DEVICE", "0")))
    yield r
    r.close()
