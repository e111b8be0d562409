"""Ported from the reference's tests/test_imports.py:4-9."""

from __future__ import annotations


def test_import_tiledattention() -> None:
    import tiledattention_amd

    assert isinstance(tiledattention_amd.__version__, str)
    assert tiledattention_amd.__version__
    assert hasattr(tiledattention_amd, "sdpa")
