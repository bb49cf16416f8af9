import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def amd_lib():
    """The in-tree libloom_accel_amd.so; built here only if nothing is built."""
    from loom_amd import _lib, build
    if not os.path.exists(_lib.LIB_PATH):
        build.build()
    return _lib.lib()


@pytest.fixture
def tuning():
    """Sets LOOM_AMD_* tuning variables for one test: tuning(name, value)
    (value None unsets).  The library reads them once and again on
    loom_amd_reload_tuning(), which this fixture calls after every change and
    after restoring the variables at the end of the test."""
    saved = {}

    def reload():
        from loom_amd import _lib
        _lib.lib().loom_amd_reload_tuning()

    def set_(name, value):
        if name not in saved:
            saved[name] = os.environ.get(name)
        if value is None:
            os.environ.pop(name, None)
        else:
            os.environ[name] = str(value)
        reload()

    yield set_
    for name, old in saved.items():
        if old is None:
            os.environ.pop(name, None)
        else:
            os.environ[name] = old
    if saved:
        reload()
