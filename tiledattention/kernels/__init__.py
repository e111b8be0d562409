"""Kernel entry points."""

from __future__ import annotations

from .flash_fwd import run_flash_fwd

__all__ = ["run_flash_fwd"]
