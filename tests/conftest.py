import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs the MI355X (gfx950) device")
    config.addinivalue_line("markers", "slow: long-running (full-size model) test")


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    d = os.environ.get("CMOL_MODEL_DIR")
    if d:
        os.makedirs(d, exist_ok=True)
        return d
    return str(tmp_path_factory.mktemp("models"))


@pytest.fixture(scope="session")
def gpu():
    """Fails (does not skip) when no device is visible: GPU tests must run
    the native path."""
    import libcmol_amd.native as native
    n = native.device_count()
    assert n >= 1, "no GPU visible to libcmol.so"
    return native
