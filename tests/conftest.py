import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libaurora_hip.so")


@pytest.fixture(scope="session")
def ctx():
    """One GpuContext per test session (the reference's tests create one per
    test and skip without an adapter; here the `gpu` marker selects the runs
    that have a GPU, so a missing device is an error, not a skip)."""
    from aurora_amd.gpu import GpuContext

    c = GpuContext.new(0)
    print(f"[gpu] device: {c.device_info()}", flush=True)
    yield c
    c.destroy()
