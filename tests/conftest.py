"""Shared pytest configuration: the ``gpu`` marker and seeded input helpers."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built native extension")


def seeded_normal(seed: int, n: int, dtype=np.float32) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal(n, dtype=np.float32).astype(dtype)


@pytest.fixture
def gpu_runtime():
    """The HIP runtime; a GPU test fails loudly (no silent fallback) when it is unusable."""
    from easy_as_amd.runtime import get_runtime

    rt = get_runtime("hip")
    return rt


@pytest.fixture(autouse=True)
def _clean_env(monkeypatch: pytest.MonkeyPatch):
    for k in ("EAS_DISABLE_THREAD_ID_REWRITE", "EAS_BACKEND"):
        monkeypatch.delenv(k, raising=False)
    yield
