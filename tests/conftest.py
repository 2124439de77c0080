import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    """The GPU; a gpu-marked test fails loudly without one (no fallback)."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible: gpu-marked tests need an MI355X")
    return torch.device("cuda:0")
