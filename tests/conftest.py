import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "vd-ttfs_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs the HIP kernels")
    config.addinivalue_line("markers", "slow: larger CPU oracle runs")


@pytest.fixture(scope="session")
def gpu_ctx_factory():
    """Creates vdttfs contexts on device 0 and closes them at session end."""
    import vdttfs

    if vdttfs.device_count() < 1:
        pytest.fail("gpu test selected but no HIP device is visible")
    made = []

    def make(consts):
        c = vdttfs.Context(consts, 0)
        made.append(c)
        return c

    yield make
    for c in made:
        c.close()
