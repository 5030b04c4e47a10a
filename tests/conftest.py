"""Test configuration: import paths, the ``gpu`` marker and shared helpers."""
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
for p in (ROOT / "colabfold-legacy-kernels_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built library")


@pytest.fixture
def cuda():
    """The ROCm device for a GPU test; skips only when this machine has no GPU at all."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device on this machine")
    return torch.device("cuda:0")
