"""Shared pytest setup.

Markers:
  gpu — needs an AMD MI355X (gfx950) GPU and the built libfa_gfx950.so; the
        driver runs these with ``-m gpu`` on a GPU box and ``-m "not gpu"`` here.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PACKAGE_ROOT = ROOT / "triton-flash-attention_amd"
for path in (str(ROOT), str(PACKAGE_ROOT)):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: requires an AMD MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    # A GPU test on a machine without a GPU is skipped with a clear reason
    # rather than failing on import-time device queries.
    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover - torch import problems surface elsewhere
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="requires an AMD MI355X (gfx950) GPU")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
