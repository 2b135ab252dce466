import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libshadowkv_amd.so")


@pytest.fixture(scope="session")
def gpu():
    """Device for GPU tests; fails (not skips) when no GPU or library is present."""
    import torch
    from shadowkv_amd import _lib

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    _lib.lib()  # raises if libshadowkv_amd.so is not built
    return torch.device("cuda:0")
