import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); calls the native library")


@pytest.fixture(scope="session")
def ctx():
    from emufpga_amd.device import Context
    c = Context(0)
    yield c
    c.close()
