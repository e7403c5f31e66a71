import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def gpu():
    """The GPU test environment: torch on cuda:0 plus the loaded HIP library.

    Loading failures raise (no fallback path exists)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from taraference_amd import capi

    capi.load()
    torch.cuda.set_device(0)
    return capi


@pytest.fixture(autouse=True)
def _release_device_buffers():
    yield
    mod = sys.modules.get("_gpu")
    if mod is not None and mod.KEEP:
        import torch

        torch.cuda.synchronize()
        mod.KEEP.clear()
