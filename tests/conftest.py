import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def gpu_present() -> bool:
    try:
        import torch  # noqa: F401  (device count only; does not initialise HIP)
        return torch.cuda.device_count() > 0
    except Exception:
        return False


@pytest.fixture(scope="session")
def hip():
    """The product C-ABI library (rustyllm_amd); GPU tests fail loudly if it is
    missing instead of falling back to anything."""
    if not gpu_present():
        pytest.skip("no GPU visible")
    from rustyllm_amd import hip as hipmod
    assert hipmod.available(), "librusty_hip.so loaded but rusty_hip_available() returned 0"
    return hipmod


@pytest.fixture(autouse=True)
def _fresh_weight_cache(request):
    """numpy may hand a freed array's address to the next test's weights; the
    library caches device copies by host address, so drop them per test."""
    if request.node.get_closest_marker("gpu") is not None and gpu_present():
        from rustyllm_amd import hip as hipmod
        hipmod.weight_cache_clear()
    yield
