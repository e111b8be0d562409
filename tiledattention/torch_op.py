"""``torch.ops.tiledattention.sdpa_fwd``: the forward as a PyTorch custom operator.

The operator is C++ (``tiledattention_amd/csrc/torch_ext.cpp``, built into
``libtiledattn_torch.so``): its schema is defined with ``TORCH_LIBRARY(tiledattention, m)``
and its implementation registered on the GPU dispatch key, so libtorch / TorchScript callers
reach it without Python, and a call from Python costs no ctypes hop.  Importing this module
loads that library (``DependencyError`` if it is missing; no fallback) and registers the
fake kernel for tracers (``torch.compile``, ``make_fx``): the same shape and dtype checks as
``sdpa`` and an empty tensor of the output's shape, dtype and device.

Schema: ``sdpa_fwd(Tensor q, Tensor k, Tensor v, bool causal=False, float? scale=None,
int tile_m=0, int tile_n=0, int accum=-1) -> Tensor``.  ``tile_m``/``tile_n`` = 0 and
``accum`` = -1 take the ``TILEDATTN_TILE_M/N`` and ``TILEDATTN_ACCUM_MODE`` knobs, as
``sdpa`` does; explicit values (tiles 64 or 128, accum 0 = fp32, 1 = the input dtype)
override them for this call, so a compiled graph does not depend on the environment.  The
C++ implementation plans the call through the library's ``ta_plan_call``, the same rules
``sdpa`` applies, so both launch the same kernel with the same arguments.

It takes the role of the reference's torch extension registration
(``torch-ext/torch_binding.cpp:6-19``, whose op is a placeholder).  Gradients are not
defined (the reference path is forward-only).  Errors of the C++ implementation carry the
messages ``sdpa`` raises, as ``RuntimeError`` (argument and knob errors as ``ValueError``).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._errors import DependencyError, InvalidShapeError
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


def _load_native_operator() -> None:
    """Load libtiledattn_torch.so once (it registers the operator with torch)."""
    if hasattr(torch.ops.tiledattention, "sdpa_fwd"):
        return
    path = _lib.lib_dir() / "libtiledattn_torch.so"
    if not path.exists():
        raise DependencyError(
            f"Native operator library {path} is missing. Build it with "
            "`python -m tiledattention_amd.csrc.build`."
        )
    _lib.load()  # the C-ABI library the operator links, loaded from the same directory
    try:
        torch.ops.load_library(str(path))
    except OSError as exc:
        raise DependencyError(f"Native operator library {path} could not be loaded: {exc}") from exc


_load_native_operator()


def sdpa_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
             scale: Optional[float] = None, tile_m: int = 0, tile_n: int = 0,
             accum: int = -1) -> torch.Tensor:
    """softmax(q k^T * scale [+ causal mask]) v for [B, H, S, D] fp16/bf16 on a gfx950 GPU,
    through the C++ operator."""
    return torch.ops.tiledattention.sdpa_fwd(q, k, v, causal, scale, tile_m, tile_n, accum)


@torch.library.register_fake(OP_NAME)
def _sdpa_fwd_fake(q, k, v, causal=False, scale=None, tile_m=0, tile_n=0, accum=-1):
    if not isinstance(causal, bool):
        raise InvalidShapeError("causal must be a bool.")
    _overrides(tile_m, tile_n, accum)
    validate_sdpa_inputs(torch, q, k, v)
    return torch.empty_like(q, memory_format=torch.contiguous_format)
