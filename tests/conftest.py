"""pytest setup: the `gpu` marker, and the import paths of the package and the oracle.

    python -m pytest tests -m "not gpu"   # oracle pins, host logic, C-ABI exports (no GPU)
    python -m pytest tests -m gpu         # HIP kernels against the oracle (needs an MI355X)
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "int8-linear_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and runs the HIP kernels")


def gpu_available() -> bool:
    import torch
    return torch.cuda.is_available()


@pytest.fixture(autouse=True)
def _skip_gpu_tests_without_gpu(request):
    if request.node.get_closest_marker("gpu") and not gpu_available():
        pytest.skip("needs a HIP GPU")
