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


def pytest_terminal_summary(terminalreporter):
    """The achieved errors of the parity checks that ran (tests/harness.py MARGINS): per test the
    worst bf16 max-abs error and cosine against the 2e-2 / 0.9995 bar, and the worst fp32 relative
    error against 1e-4 -- the margins, printed even under -q."""
    try:
        import harness
    except Exception:
        return
    if not harness.MARGINS:
        return
    worst = {}
    for test, what, kind, err, cos in harness.MARGINS:
        k = (test, kind)
        e0, c0 = worst.get(k, (0.0, 1.0))
        worst[k] = (max(e0, err), min(c0, cos) if cos is not None else c0)
    tr = terminalreporter
    tr.write_sep("-", "parity margins (worst per test)")
    for (test, kind), (err, cos) in sorted(worst.items(), key=lambda kv: (kv[0][1], kv[1][0] / (2e-2 if kv[0][1] == "bf16" else 1e-4))):
        if kind == "bf16":
            tr.write_line("bf16 %-58s max-abs %.4f (bar 2e-2)  cosine %.7f" % (test[:58], err, cos))
        else:
            tr.write_line("fp32 %-58s rel %.2e (bar 1e-4)" % (test[:58], err))
    b = [v for (t, k), v in worst.items() if k == "bf16"]
    f = [v for (t, k), v in worst.items() if k == "fp32"]
    if b:
        tr.write_line("bf16 overall: worst max-abs %.4f of 2e-2, lowest cosine %.7f (%d tests)"
                      % (max(e for e, _ in b), min(c for _, c in b), len(b)))
    if f:
        tr.write_line("fp32 overall: worst relative error %.2e of 1e-4 (%d tests)" % (max(e for e, _ in f), len(f)))

