"""Shared pytest setup.

Marker `gpu`: needs an MI355X.  When no GPU is visible these tests are skipped,
unless the run explicitly selects them (`-m gpu`), in which case they run and
fail loudly -- a GPU run must never pass by skipping.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
# kernel arguments in device memory, as the Python binding sets it, also for the C++
# test programs started before the library is loaded here
os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "1")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test needs an AMD GPU (MI355X / gfx950)")


def _gpu_visible() -> bool:
    try:
        from kvcache_amd.device import has_device
        return has_device()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    markexpr = (config.option.markexpr or "").replace(" ", "")
    explicitly_gpu = "gpu" in markexpr and "notgpu" not in markexpr
    if explicitly_gpu or _gpu_visible():
        return
    skip = pytest.mark.skip(reason="no GPU visible (run with -m gpu on an MI355X)")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.build()
    return oracle
