import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) HIP device")
    # Load the encoder library (and with it the system HIP runtime) before any test module is
    # imported, so the process binds libamdhip64 to the runtime the library was built against.
    try:
        load_pkg().load_library()
    except Exception:
        pass


def load_pkg():
    """Imports universal-dictator_amd/ (a hyphenated directory) as module universal_dictator_amd."""
    name = "universal_dictator_amd"
    if name in sys.modules:
        return sys.modules[name]
    path = os.path.join(ROOT, "universal-dictator_amd", "__init__.py")
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def ud():
    return load_pkg()


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def gpu(ud):
    """The library with a HIP device; GPU tests fail (not skip) when it is missing."""
    ud.lib()
    return ud
