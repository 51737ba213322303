"""Test tiers: CPU tests (oracle pins, C-ABI surface, host logic) run anywhere;
tests marked ``gpu`` need an MI355X and call the HIP kernels through the C ABI."""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X / gfx950)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def _gpu_count() -> int:
    import strict_amd

    return strict_amd.device_count()


@pytest.fixture(scope="session")
def ctx():
    """One libstrict_hip context on device 0 for the whole GPU session."""
    import strict_amd

    if _gpu_count() == 0:
        pytest.skip("no HIP device visible")
    c = strict_amd.Context(0)
    info = c.info()
    print(f"\n[gpu] {info['name']} {info['arch']} CUs={info['compute_units']}", flush=True)
    yield c
    c.dispose()


@pytest.fixture(scope="session")
def rng_seed() -> int:
    return int(os.environ.get("STRICT_SEED", "42"))
