"""MI355X-native SDPA forward with the public API of TiledAttention.

``sdpa(q, k, v, *, causal=False, scale=None) -> o`` on [B, H, S, D] fp16/bf16 tensors,
backed by hand-written gfx950 HIP kernels behind a C ABI (``include/tiledattn.h``).
The names exported here match ``src/tiledattention/__init__.py:47-55`` of the reference.
"""

from __future__ import annotations

from typing import TYPE_CHECKING

from ._errors import (
    DependencyError,
    DTypeNotSupportedError,
    InvalidShapeError,
    TiledAttentionError,
    UnsupportedPlatformError,
)
from ._version import __version__

if TYPE_CHECKING:
    import torch


def sdpa(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    causal: bool = False,
    scale: float | None = None,
) -> torch.Tensor:
    """Scaled dot-product attention forward; see ``tiledattention.sdpa.sdpa``."""
    from .sdpa import sdpa as _sdpa

    return _sdpa(q, k, v, causal=causal, scale=scale)


__all__ = [
    "__version__",
    "sdpa",
    "TiledAttentionError",
    "UnsupportedPlatformError",
    "InvalidShapeError",
    "DTypeNotSupportedError",
    "DependencyError",
]
