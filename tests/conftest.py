import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "p40-kernel_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    path = os.path.join(ROOT, "tests", "golden", "golden.npz")
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture
def knobs(monkeypatch):
    """Set or clear the library's BONSAI_* tuning variables for one test.  The
    library reads them once per process, so every change is followed by
    bonsai_p40_reload_tuning(), and the previous environment is restored and
    re-read when the test ends."""
    import bonsai_p40 as B

    class Knobs:
        def set(self, name, value):
            monkeypatch.setenv(name, str(value))
            B.reload_tuning()

        def unset(self, name):
            monkeypatch.delenv(name, raising=False)
            B.reload_tuning()

    yield Knobs()
    monkeypatch.undo()
    B.reload_tuning()
