"""Input-contract helpers."""

from __future__ import annotations

from .checks import validate_sdpa_inputs

__all__ = ["validate_sdpa_inputs"]
