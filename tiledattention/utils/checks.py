"""q/k/v contract checks, in the reference's order and with its messages.

Reference: ``src/tiledattention/utils/checks.py:10-55``. The order matters because
tests pin which error wins when several are wrong at once:

1. each of q, k, v is a ``torch.Tensor``;
2. per tensor: 4 dims, then on the GPU (``is_cuda`` is True for HIP tensors on
   PyTorch-ROCm);
3. equal shapes (no cross-attention, no GQA), then equal devices;
4. dtype in {float16, bfloat16}, then equal dtypes.
"""

from __future__ import annotations

from types import ModuleType

from .._errors import DTypeNotSupportedError, InvalidShapeError


def _ensure_tensor(torch_mod: ModuleType, name: str, value: object) -> None:
    """Raise ``InvalidShapeError`` unless ``value`` is a tensor of ``torch_mod``."""
    if not isinstance(value, torch_mod.Tensor):
        raise InvalidShapeError(f"{name} must be a torch.Tensor.")


def validate_sdpa_inputs(torch_mod: ModuleType, q, k, v) -> None:
    """Check the SDPA input contract; raise the first violation found."""
    tensor_type = torch_mod.Tensor
    if type(q) is tensor_type and type(k) is tensor_type and type(v) is tensor_type:
        # Every check below at once (plain tensors, 4-d, one shape, one CUDA device, one
        # dtype in {fp16, bf16}); any failure takes the ordered checks for its message.
        shape, dev, dt = q.shape, q.device, q.dtype
        if (len(shape) == 4 and q.is_cuda and k.is_cuda and v.is_cuda and shape == k.shape
                and shape == v.shape and dev == k.device and dev == v.device
                and (dt is torch_mod.float16 or dt is torch_mod.bfloat16)
                and dt == k.dtype and dt == v.dtype):
            return
    _ensure_tensor(torch_mod, "q", q)
    _ensure_tensor(torch_mod, "k", k)
    _ensure_tensor(torch_mod, "v", v)

    for name, tensor in (("q", q), ("k", k), ("v", v)):
        if tensor.ndim != 4:
            raise InvalidShapeError(f"{name} must have shape [B, H, S, D].")
        if not bool(tensor.is_cuda):
            raise InvalidShapeError(f"{name} must be a CUDA tensor.")

    if q.shape != k.shape or q.shape != v.shape:
        raise InvalidShapeError("q, k, and v must have matching shape [B, H, S, D].")

    if q.device != k.device or q.device != v.device:
        raise InvalidShapeError("q, k, and v must be on the same CUDA device.")

    allowed_dtypes = {torch_mod.float16, torch_mod.bfloat16}
    if q.dtype not in allowed_dtypes:
        raise DTypeNotSupportedError("q dtype must be torch.float16 or torch.bfloat16.")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise DTypeNotSupportedError("q, k, and v must have identical dtype.")
