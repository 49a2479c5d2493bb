import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


_DEV = None


def gpu_device():
    """One shared HIP context for the GPU tests (one process, one context)."""
    global _DEV
    if _DEV is None:
        import intfer_amd as ia
        try:
            _DEV = ia.Device(0)
        except ia.IfrError as e:
            pytest.skip(f"no usable GPU: {e}")
    return _DEV


@pytest.fixture(scope="session")
def dev():
    d = gpu_device()
    yield d


def announce(msg: str) -> None:
    """Name the case before a GPU step, flushed (so a lost box still says what ran)."""
    sys.stdout.write(f"[case] {msg}\n")
    sys.stdout.flush()
