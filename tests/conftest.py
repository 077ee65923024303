"""pytest configuration: the `gpu` marker and the import path.

Tests that need an MI355X carry @pytest.mark.gpu. Without a GPU they are skipped, unless the run selects them
explicitly (-m gpu), in which case they run and fail loudly instead of passing on nothing.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950) and the built libbyteprof_amd.so")


def pytest_collection_modifyitems(config, items):
    markexpr = config.getoption("-m") or ""
    if "gpu" in markexpr and "not gpu" not in markexpr:
        return
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="needs a GPU (run with -m gpu on an MI355X)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
