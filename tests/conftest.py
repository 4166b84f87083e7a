import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "oracle")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    import pyoracle
    return pyoracle.load_oracle()


@pytest.fixture(scope="session")
def ref():
    import pyoracle
    if not pyoracle.ref_available():
        pytest.skip("reference CPU library (oracle/_ref) is not built here")
    return pyoracle.load_ref()
