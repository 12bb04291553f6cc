import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); parity tests proper")
    config.addinivalue_line("markers", "slow: longer CPU tests")


@pytest.fixture
def rng():
    # The reference's shared fixture (tests/conftest.py:21-23).
    return np.random.default_rng(seed=17)


def _has_gpu() -> bool:
    try:
        from palladium_amd import runtime

        return runtime.device_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords and os.environ.get("PALLADIUM_REQUIRE_GPU") != "1":
            item.add_marker(skip)
