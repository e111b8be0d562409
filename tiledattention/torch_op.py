"""``torch.ops.tiledattention.sdpa_fwd``: the forward as a PyTorch custom operator.

Importing this module registers the operator (``torch.library.custom_op``) with a fake
kernel, so ``torch.compile`` and other tracers can place it in a graph without running it:
the fake applies the same shape and dtype checks as ``sdpa`` and returns an empty tensor of
the output's shape, dtype and device.  The real kernel is ``tiledattention.sdpa``'s path
(the gfx950 HIP kernels; no fallback).

Schema: ``sdpa_fwd(Tensor q, Tensor k, Tensor v, bool causal=False, float? scale=None,
int tile_m=0, int tile_n=0, int accum=-1) -> Tensor``.  ``tile_m``/``tile_n`` = 0 and
``accum`` = -1 take the ``TILEDATTN_TILE_M/N`` and ``TILEDATTN_ACCUM_MODE`` knobs, as
``sdpa`` does; explicit values (tiles 64 or 128, accum 0 = fp32, 1 = the input dtype)
override them for this call, so a compiled graph does not depend on the environment.

It takes the role of the reference's torch extension registration
(``torch-ext/torch_binding.cpp:6-19``, whose op is a placeholder) for callers that want an
operator rather than a Python function.  Gradients are not defined (the reference path is
forward-only).
"""

from __future__ import annotations

from typing import Optional

import torch

from ._errors import InvalidShapeError
from .sdpa import _sdpa_checked
from .utils.checks import validate_sdpa_inputs

__all__ = ["sdpa_fwd", "OP_NAME"]

OP_NAME = "tiledattention::sdpa_fwd"

_ACCUM_NAMES = {0: "fp32", 1: "fp16"}


def _overrides(tile_m: int, tile_n: int, accum: int) -> dict:
    """Keyword overrides for ``run_flash_fwd`` from the operator's integer arguments."""
    out: dict = {}
    if (tile_m == 0) != (tile_n == 0):
        raise ValueError("tile_m and tile_n must both be 0 (use the knobs) or both be given.")
    if tile_m:
        if tile_m not in (64, 128) or tile_n not in (64, 128):
            raise ValueError(f"Unsupported tile ({tile_m}, {tile_n}): tiles are 64 or 128.")
        out["tile"] = (int(tile_m), int(tile_n))
    if accum != -1:
        if accum not in _ACCUM_NAMES:
            raise ValueError(f"accum must be -1 (knob), 0 (fp32) or 1 (input dtype), got {accum}.")
        out["accum"] = _ACCUM_NAMES[accum]
    return out


@torch.library.custom_op(OP_NAME, mutates_args=())
def sdpa_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
             scale: Optional[float] = None, tile_m: int = 0, tile_n: int = 0,
             accum: int = -1) -> torch.Tensor:
    """softmax(q k^T * scale [+ causal mask]) v for [B, H, S, D] fp16/bf16 on a gfx950 GPU."""
    out = _sdpa_checked(q, k, v, causal=causal, scale=scale, **_overrides(tile_m, tile_n, accum))
    # A padded head dim comes back as a column slice of a wider buffer; an operator's output
    # must own its storage layout, so return it dense.
    return out if out.is_contiguous() else out.contiguous()


@sdpa_fwd.register_fake
def _sdpa_fwd_fake(q, k, v, causal=False, scale=None, tile_m=0, tile_n=0, accum=-1):
    if not isinstance(causal, bool):
        raise InvalidShapeError("causal must be a bool.")
    _overrides(tile_m, tile_n, accum)
    validate_sdpa_inputs(torch, q, k, v)
    return torch.empty_like(q, memory_format=torch.contiguous_format)
