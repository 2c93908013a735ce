import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.join(ROOT, "tests")
PKG = os.path.join(ROOT, "phonon-2-c_amd")
for p in (TESTS, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


import pytest  # noqa: E402


class _SwitchMonkeyPatch(pytest.MonkeyPatch):
    """monkeypatch whose environment changes to the library's P2H_* switches take effect: the library reads them once
    at initialisation, so each change (and the undo at the end of the test) is followed by p2h_reload_switches."""

    def _reload(self, name):
        if str(name).startswith("P2H_"):
            import p2gemm
            p2gemm.reload_switches()

    def setenv(self, name, value, prepend=None):
        super().setenv(name, value, prepend)
        self._reload(name)

    def delenv(self, name, raising=True):
        super().delenv(name, raising)
        self._reload(name)

    def undo(self):
        names = [k for (_, k, _) in self._setitem if k is not None] if hasattr(self, "_setitem") else []
        super().undo()
        if any(str(k).startswith("P2H_") for k in names):
            import p2gemm
            p2gemm.reload_switches()


@pytest.fixture
def monkeypatch():
    mp = _SwitchMonkeyPatch()
    yield mp
    mp.undo()
