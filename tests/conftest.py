"""Test configuration: the ``gpu`` marker and the repository root on ``sys.path``.

``gpu`` tests need a HIP device (an MI355X). Without one they are skipped, or,
with ``AYAKA_REQUIRE_GPU=1``, they fail (reference ``tests/conftest.py:1-56``).
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built library")


def _have_gpu() -> bool:
    try:
        import torch
    except ImportError:
        return False
    return bool(torch.cuda.is_available() and torch.version.hip is not None)


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    if _have_gpu() or os.environ.get("AYAKA_REQUIRE_GPU") == "1":
        return  # run them; without a device they fail
    skip = pytest.mark.skip(reason="needs a HIP device")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
