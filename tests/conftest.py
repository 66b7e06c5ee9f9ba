import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")


@pytest.fixture(scope="session")
def hip():
    """The initialised HIP device.  A GPU test fails (not skips) when the
    device or the library is missing: the product has no CPU path."""
    import thvm_amd
    os.environ.setdefault("THVM_HIP_CACHE_DIR", str(ROOT / "gpurun_out" / "hip_co_cache"))
    thvm_amd.init()
    yield thvm_amd
    thvm_amd.shutdown()
