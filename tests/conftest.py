import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libullis_hip.so)")


@pytest.fixture(scope="session")
def rt():
    from ullis_amd.runtime import HipRuntime

    r = HipRuntime(0)  # raises (no skip) when the library or the GPU is missing
    yield r
    r.close()
