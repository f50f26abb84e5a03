import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an AMD Instinct GPU (gfx950) and the built HIP library"
    )


def gpu_available() -> bool:
    return torch.cuda.is_available() and torch.version.hip is not None


@pytest.fixture(scope="session")
def native_lib():
    """The loaded C-ABI library; a missing or broken library fails the test loudly."""
    from muspace_amd.runtime import native

    return native.load_native_module()
