import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU")


@pytest.fixture(scope="session")
def orc():
    import pyoracle
    return pyoracle.Oracle()


@pytest.fixture(scope="session")
def ref():
    import pyoracle
    if not pyoracle.Ref.available():
        pytest.skip("reference build oracle/_ref not present here")
    return pyoracle.Ref()


@pytest.fixture(scope="session")
def gctx():
    """ftx context on device 0.  The GPU tests must run the HIP library: a
    missing library or device is an error, not a skip."""
    from xwfes_amd import ftx
    ctx = ftx.Context(0)
    yield ctx
    ctx.close()
