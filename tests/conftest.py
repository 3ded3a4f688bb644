"""Shared pytest setup.

* puts the package (``causal-conv1d-mojo_amd/``) and the repo root (for the
  ``oracle`` test package) on ``sys.path``;
* registers the ``gpu`` marker; GPU tests are skipped when no ROCm device is
  visible, so ``pytest -m "not gpu"`` and a GPU-less ``pytest`` both run;
* seeds torch before every test (as the reference's ``tests/conftest.py:32-36``).
"""

from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "causal-conv1d-mojo_amd", ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import pytest  # noqa: E402
import torch  # noqa: E402

HAS_GPU = torch.version.hip is not None and torch.cuda.is_available()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    if HAS_GPU:
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _seed_rng():
    torch.manual_seed(0)
    if HAS_GPU:
        torch.cuda.manual_seed_all(0)
