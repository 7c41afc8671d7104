import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; parity tests proper")


@pytest.fixture(scope="session")
def device():
    """The GPU, through libkvattn (fails loudly when the library is missing)."""
    from mi50grad_amd.device import GPUDevice, device_count

    assert device_count() >= 1, "no GPU visible to libkvattn"
    dev = GPUDevice(0)
    yield dev
    dev.cleanup()
