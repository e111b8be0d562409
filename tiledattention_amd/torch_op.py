"""``torch.ops.tiledattention.sdpa_fwd``: the forward as a PyTorch custom operator.

Importing this module registers the operator (``torch.library.custom_op``) with a fake
kernel, so ``torch.compile`` and other tracers can place it in a graph without running it:
the fake applies the same shape and dtype checks as ``sdpa`` and returns an empty tensor of
the output's shape, dtype and device.  The real kernel is ``tiledattention_amd.sdpa`` (the
gfx950 HIP path; no fallback).

It takes the role of the reference's torch extension registration
(``torch-ext/torch_binding.cpp:6-19``, whose op is a placeholder) for callers that want an
operator rather than a Python function.  Gradients are not defined (the reference path is
forward-only).
"""

from __future__ import annotations

from typing import Optional

import torch

from .sdpa import sdpa as _sdpa
from .utils.checks import validate_sdpa_inputs

__all__ = ["sdpa_fwd", "OP_NAME"]

OP_NAME = "tiledattention::sdpa_fwd"


@torch.library.custom_op(OP_NAME, mutates_args=())
def sdpa_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
             scale: Optional[float] = None) -> torch.Tensor:
    """softmax(q k^T * scale [+ causal mask]) v for [B, H, S, D] fp16/bf16 on a gfx950 GPU."""
    out = _sdpa(q, k, v, causal=causal, scale=scale)
    # A padded head dim comes back as a column slice of a wider buffer; an operator's output
    # must own its storage layout, so return it dense.
    return out if out.is_contiguous() else out.contiguous()


@sdpa_fwd.register_fake
def _sdpa_fwd_fake(q, k, v, causal=False, scale=None):
    if not isinstance(causal, bool):
        raise TypeError("causal must be a bool.")
    validate_sdpa_inputs(torch, q, k, v)
    return torch.empty_like(q, memory_format=torch.contiguous_format)
