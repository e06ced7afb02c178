import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "onnxruntime-ep-vulkan_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def cuda():
    """The GPU under test.  A gpu-marked test that finds no GPU or no built library fails."""
    import torch

    assert torch.cuda.is_available(), "gpu test selected but no GPU is visible"
    import mnb

    mnb.load()
    return torch.device("cuda:0")
