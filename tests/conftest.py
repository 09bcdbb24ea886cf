import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "sam3.c_amd"))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _reload_settings():
    from sam3_amd import hip
    hip.load().sam3_hip_reload_settings()


@pytest.fixture
def env(monkeypatch):
    """Set or unset SAM3_HIP_* switches for one test. The library parses
    them once, so every change is followed by sam3_hip_reload_settings(),
    and the original environment is restored (and re-read) afterwards."""
    class Env:
        def set(self, name, value):
            monkeypatch.setenv(name, str(value))
            _reload_settings()

        def unset(self, name):
            monkeypatch.delenv(name, raising=False)
            _reload_settings()

    yield Env()
    monkeypatch.undo()
    _reload_settings()
