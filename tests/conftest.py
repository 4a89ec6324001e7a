"""Shared test setup: import paths, the `gpu` marker, and GPU tests skipping themselves on CPU machines.

Mirrors fastserve tests/conftest.py:13-25 (gpu-marked tests are skipped when no GPU is visible).
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "bytes-per-token_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _has_gpu() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except ImportError:
        return False


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="needs a GPU")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def built_lib():
    """The library, built in-tree first if nothing is built yet. A library built from other sources than the
    tree's is refused (StaleLibraryError), failing every test that uses it."""
    from bpt_amd import _build, _lib

    if not _lib.LIB_PATH.exists():
        _build.build()
    return _lib.lib()
