import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device; runs the HIP kernels")
    config.addinivalue_line("markers", "slow: large inputs (hundreds of MB)")


@pytest.fixture(scope="session")
def ctx():
    """One gfx950 context for the whole GPU session. Fails (does not skip) without a device:
    GPU tests are only collected with -m gpu on the GPU box, where a missing device is an error."""
    from dotcompute_amd import hip

    n = hip.device_count()
    assert n >= 1, "no HIP device visible"
    info = hip.device_info(0)
    print(f"\n[gpu] device 0: {info.name.decode()} {info.gcn_arch_name.decode()} CUs={info.compute_units}", flush=True)
    c = hip.Context(0)
    yield c
    c.close()
