"""Exception hierarchy of the SDPA operator.

Mirrors ``src/tiledattention/_errors.py:6-23`` of the reference: one base class and
four subclasses with the same names, so callers that catch the reference's errors
keep working unchanged.
"""

from __future__ import annotations


class TiledAttentionError(Exception):
    """Base class of every error this package raises on purpose."""


class UnsupportedPlatformError(TiledAttentionError):
    """The process cannot run the operator here (no HIP device, wrong GPU arch)."""


class InvalidShapeError(TiledAttentionError):
    """q/k/v (or ``causal``/``scale``) break the operator's input contract."""


class DTypeNotSupportedError(TiledAttentionError):
    """Input dtype is neither float16 nor bfloat16, or q/k/v dtypes differ."""


class DependencyError(TiledAttentionError):
    """A required component is missing: torch, the C-ABI library or a code object."""
