"""Shared test setup.

Markers: ``gpu`` - needs a gfx950 GPU and the built native library; the CPU suite runs with
``-m "not gpu"``.  The repository root is put on ``sys.path`` so ``oracle`` (test
infrastructure) and ``tiledattention`` import from the checkout.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

_KNOBS = (
    "TILEDATTN_TILE_M",
    "TILEDATTN_TILE_N",
    "TILEDATTN_ACCUM_MODE",
    "TILEDATTN_SYNC_MODE",
    "TILEDATTN_DISABLE_ALIGNED_FASTPATH",
    "TILEDATTN_KERNEL_OPT_LEVEL",
    "TILEDATTN_KERNEL_OCCUPANCY",
    "TILEDATTN_KERNEL_NUM_CTAS",
    "TILEDATTN_CHUNKED_HEAD_DIMS",
    "TILEDATTN_SCHED",
)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP kernels")


@pytest.fixture(autouse=True)
def _clean_knobs(monkeypatch):
    """Every test starts with the operator's env knobs unset."""
    for name in _KNOBS:
        monkeypatch.delenv(name, raising=False)
    yield


def gpu_available() -> bool:
    try:
        import torch
    except ImportError:
        return False
    return bool(torch.cuda.is_available())


@pytest.fixture
def gpu():
    """Skip unless a GPU is visible; on a GPU box the kernels must be built (fail loudly)."""
    if not gpu_available():
        pytest.skip("no GPU visible")
    from tiledattention import _runtime

    _runtime._reset_runtime_cache_for_tests()
    _runtime.require_supported_runtime()
    import torch

    return torch.device("cuda:0")

