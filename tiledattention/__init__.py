"""MI355X-native SDPA forward with the public API of TiledAttention.

``sdpa(q, k, v, *, causal=False, scale=None) -> o`` on [B, H, S, D] fp16/bf16 tensors,
backed by hand-written gfx950 HIP kernels behind a C ABI (``include/tiledattn.h``).
The names exported here match ``src/tiledattention/__init__.py:47-55`` of the reference.
"""

from __future__ import annotations

import importlib as _importlib
import sys as _sys
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
    # The submodule's current ``sdpa`` on every call (as the reference's per-call import
    # resolves it), found in sys.modules once it is imported.
    mod = _sys.modules.get(_SDPA_MODULE)
    if mod is None:
        mod = _importlib.import_module(_SDPA_MODULE)
    return mod.sdpa(q, k, v, causal=causal, scale=scale)


_SDPA_MODULE = __name__ + ".sdpa"


__all__ = [
    "__version__",
    "sdpa",
    "TiledAttentionError",
    "UnsupportedPlatformError",
    "InvalidShapeError",
    "DTypeNotSupportedError",
    "DependencyError",
]
