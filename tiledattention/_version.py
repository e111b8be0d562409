"""Package version (reference: ``src/tiledattention/_version.py:8-22``)."""

from __future__ import annotations

from importlib.metadata import PackageNotFoundError, version


def _resolve_version() -> str:
    """Installed distribution version, or ``"0.0.0"`` for an in-tree checkout."""
    try:
        return version("tiledattention")
    except PackageNotFoundError:
        return "0.0.0"


__version__ = _resolve_version()
