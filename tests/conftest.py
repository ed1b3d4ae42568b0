import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (HERE, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library on the device)")


def gpu_available():
    try:
        import torch  # noqa: F401  (device count only; does not initialise HIP)
        return torch.cuda.device_count() > 0
    except Exception:
        return False


@pytest.fixture(scope="session")
def jas():
    """The HIP library binding; GPU tests fail loudly if it is not built."""
    import jasmine_amd
    jasmine_amd.check(jasmine_amd.lib.jas_init(0))
    return jasmine_amd
