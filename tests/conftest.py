import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "tests"), os.path.join(ROOT, "sana.cpp_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

# torch ships its own HIP runtime; loaded after libsana_dit.so (which links
# the system ROCm's), it finds no GPU.  Importing torch first, before any test
# loads the library, keeps the tests that hand torch tensors to the C ABI
# working in any order or selection.
try:
    import torch  # noqa: F401
except ImportError:
    pass


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libsana_dit.so on cuda:0)")
    config.addinivalue_line("markers", "slow: long CPU oracle run")


# Relative L2 errors computed by each test, printed at the end of the session
# (also under -q), so a run's record carries the parity figures, not only pass
# counts.  Every test still asserts against its own tolerance.
_current = {"test": None}
_record = {}


@pytest.fixture(autouse=True)
def _parity_record(request):
    _current["test"] = request.node.nodeid
    yield
    _current["test"] = None


def rel_l2(a, b):
    import numpy as np
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    v = float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
    if _current["test"]:
        _record.setdefault(_current["test"], []).append(v)
    return v


def spread_subsample(arr, fx, name):
    """(got, want) at the fixture's spread indices (k * step) mod size, or None
    when the fixture has no spread subsample of `name`."""
    import numpy as np
    if name + "__spread" not in fx:
        return None
    want = fx[name + "__spread"]
    flat = np.asarray(arr).reshape(-1)
    idx = (np.arange(want.size, dtype=np.int64) * int(fx[name + "__spread_step"])) % flat.size
    return flat[idx], want


def pytest_terminal_summary(terminalreporter):
    if not _record:
        return
    # per test function (parameter sets folded): largest relative L2 and count
    agg = {}
    for nodeid, vals in _record.items():
        key = nodeid.split("[")[0].split("::")[-1]
        m, n = agg.get(key, (0.0, 0))
        agg[key] = (max(m, max(vals)), n + len(vals))
    terminalreporter.write_sep("-", "relative L2 per test function: max over its comparisons (count)")
    line = ""
    for k, (m, n) in agg.items():
        item = f"{k} {m:.2e} ({n})"
        if line and len(line) + len(item) + 2 > 160:
            terminalreporter.write_line(line)
            line = ""
        line = f"{line}; {item}" if line else item
    if line:
        terminalreporter.write_line(line)
