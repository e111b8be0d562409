"""PyTorch-facing SDPA entry point.

Same checks in the same order as the reference (src/tiledattention/sdpa.py:14-48):

1. ``causal`` must be a bool, ``scale`` None or a positive real -> ``InvalidShapeError``
   (as in the reference, ``True`` passes as 1.0 and NaN/inf pass the check);
2. runtime gate (``_runtime.require_supported_runtime``) - before any tensor check, so a
   process without a usable GPU reports that first;
3. tensor contract (``utils.checks.validate_sdpa_inputs``);
4. default scale ``1/sqrt(D)`` in double precision (D = 0 raises ``ZeroDivisionError``);
5. ``run_flash_fwd``, looked up in this module's namespace at call time so tests can
   replace it.

Unlike the reference, this module is itself callable: importing ``tiledattention.sdpa``
as a submodule rebinds the package attribute ``sdpa`` from the function to this module
(Python's import system sets the attribute on the parent package), and in the reference
that leaves ``tiledattention.sdpa`` uncallable after the first call.  Making the module
callable keeps ``package.sdpa(q, k, v)`` working either way.
"""

from __future__ import annotations

import math
import sys
import types
from numbers import Real

from . import _runtime
from ._errors import InvalidShapeError
from .kernels import run_flash_fwd
from .utils.checks import validate_sdpa_inputs


def sdpa(
    q,
    k,
    v,
    *,
    causal: bool = False,
    scale: float | None = None,
):
    """softmax(q k^T * scale [+ causal mask]) v for [B, H, S, D] fp16/bf16 GPU tensors.

    Args:
        q, k, v: tensors of identical shape [B, H, S, D], dtype and device.
        causal: mask keys after each query (key j visible to query i iff j <= i).
        scale: softmax scale; ``None`` means ``1/sqrt(D)``.

    Returns:
        o, [B, H, S, D] in the input dtype.
    """
    return _sdpa_checked(q, k, v, causal=causal, scale=scale)


def _sdpa_checked(q, k, v, *, causal, scale, **overrides):
    """``sdpa``'s checks and launch; ``overrides`` (``tile``, ``accum``) reach
    ``run_flash_fwd`` only when given, so ``sdpa`` calls it exactly as the reference does."""
    if not isinstance(causal, bool):
        raise InvalidShapeError("causal must be a bool.")
    if scale is not None and (not isinstance(scale, Real) or float(scale) <= 0):
        raise InvalidShapeError("scale must be a positive number when provided.")

    _runtime.require_supported_runtime()
    torch_mod = _runtime.get_torch_module()
    validate_sdpa_inputs(torch_mod, q, k, v)

    head_dim = int(q.shape[-1])
    resolved_scale = float(scale) if scale is not None else 1.0 / math.sqrt(head_dim)
    return run_flash_fwd(q, k, v, causal=causal, scale=resolved_scale, **overrides)


class _CallableModule(types.ModuleType):
    """Module type whose instances forward calls to this module's ``sdpa`` function."""

    def __call__(self, *args, **kwargs):
        return sdpa(*args, **kwargs)


sys.modules[__name__].__class__ = _CallableModule
