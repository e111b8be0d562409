"""Runtime gate: is this process able to run the gfx950 SDPA kernels?

Re-targets ``src/tiledattention/_runtime.py:1-205`` of the reference from CUDA/Blackwell +
CuPy + cuTile to ROCm/gfx950 + this package's C-ABI library:

=====================================  ==============================================
reference check                        here
=====================================  ==============================================
``torch.cuda.is_available()``          same (True on PyTorch-ROCm with a visible GPU)
compute capability major in {10, 12}   PyTorch built for ROCm and ``gcnArchName``
                                       starting with ``gfx950``
``import cupy``, ``import cuda.tile``  ``libtiledattn.so`` and its gfx950 code objects
                                       load (``_get_native_library``)
=====================================  ==============================================

As in the reference the gate runs once per process under a lock, errors are
``UnsupportedPlatformError`` / ``DependencyError``, and ``_reset_runtime_cache_for_tests``
clears the cached state.  The module getters are module-level functions so that tests can
monkeypatch them exactly as the reference's tests do.
"""

from __future__ import annotations

import importlib
from threading import Lock
from types import ModuleType

from ._errors import DependencyError, UnsupportedPlatformError

_SUPPORTED_ARCH_PREFIXES = ("gfx950",)
_runtime_ready = False
_runtime_lock = Lock()
_cached_torch: ModuleType | None = None
_cached_native = None


def _get_torch_module() -> ModuleType:
    """Import torch once; ``DependencyError`` if it is not installed."""
    global _cached_torch
    if _cached_torch is not None:
        return _cached_torch
    try:
        _cached_torch = importlib.import_module("torch")
        return _cached_torch
    except ModuleNotFoundError as exc:
        raise DependencyError(
            "PyTorch is required for tiledattention. Install a ROCm-enabled torch build first."
        ) from exc


def get_torch_module() -> ModuleType:
    """Public accessor used by the kernel host code and harnesses."""
    return _get_torch_module()


def _get_native_library():
    """Load the C-ABI library (and check its code objects) once per process."""
    global _cached_native
    if _cached_native is not None:
        return _cached_native
    from . import _lib

    _cached_native = _lib.load()
    return _cached_native


def get_native_library():
    """Public accessor for the loaded C-ABI library."""
    return _get_native_library()


def _query_device_arch(torch_mod: ModuleType) -> str:
    """``gcnArchName`` of the current device, e.g. ``'gfx950:sramecc+:xnack-'``."""
    try:
        device_index = torch_mod.cuda.current_device()
        props = torch_mod.cuda.get_device_properties(device_index)
        return str(getattr(props, "gcnArchName", "") or "")
    except Exception as exc:  # pragma: no cover - defensive path
        raise UnsupportedPlatformError("Unable to query the GPU architecture from torch.cuda.") from exc


def require_supported_runtime() -> None:
    """Raise unless torch sees a gfx950 GPU and the native library loads."""
    global _runtime_ready

    if _runtime_ready:  # set only after every check below has passed
        return
    with _runtime_lock:
        if _runtime_ready:
            return

        torch_mod = _get_torch_module()

        if not bool(torch_mod.cuda.is_available()):
            raise UnsupportedPlatformError(
                "tiledattention requires a ROCm (HIP) GPU of the MI355X class (gfx950). "
                "torch.cuda.is_available() is False."
            )

        hip_version = getattr(getattr(torch_mod, "version", None), "hip", None)
        if not hip_version:
            raise UnsupportedPlatformError(
                "tiledattention requires PyTorch built for ROCm (torch.version.hip is not set)."
            )

        arch = _query_device_arch(torch_mod)
        if not arch.startswith(_SUPPORTED_ARCH_PREFIXES):
            raise UnsupportedPlatformError(
                f"Unsupported GPU: architecture {arch or 'unknown'}; "
                "requires gfx950 (MI355X / MI350X class)."
            )

        _get_native_library()

        _runtime_ready = True


def _reset_runtime_cache_for_tests() -> None:
    """Forget every cached module and the ready flag (tests swap fakes in)."""
    global _runtime_ready, _cached_torch, _cached_native
    with _runtime_lock:
        _runtime_ready = False
        _cached_torch = None
        _cached_native = None
