"""Process-wide cache of ready-to-launch kernels.

Keeps the interface of ``src/tiledattention/kernels/compile_cache.py:10-37``:
``get_kernel(key, factory)`` returns the cached callable for ``key`` or builds it with
``factory()``, and ``reset_cache_for_tests()`` empties the cache.  Differences:

* the factory does not JIT-compile anything: it asks the C-ABI library to load the
  precompiled gfx950 code object for the key and resolve the kernel symbol
  (``ta_prepare``), which the library caches per device behind its own mutex;
* the Python dict is guarded by a lock (the reference's is not);
* ``reset_cache_for_tests()`` also unloads the library's modules (``ta_cache_reset``).
"""

from __future__ import annotations

from collections.abc import Callable
from threading import Lock

KernelCallable = Callable[..., object]
KernelKey = tuple[object, ...]

_KERNEL_CACHE: dict[KernelKey, KernelCallable] = {}
_CACHE_LOCK = Lock()
_generation = 0  # bumped by every reset; callers holding kernels across calls compare it


def get_kernel(key: KernelKey, factory: Callable[[], KernelCallable]) -> KernelCallable:
    """Return the cached kernel for ``key``, creating it with ``factory`` on a miss."""
    with _CACHE_LOCK:
        kernel = _KERNEL_CACHE.get(key)
        if kernel is None:
            kernel = factory()
            _KERNEL_CACHE[key] = kernel
        return kernel


def cache_size() -> int:
    with _CACHE_LOCK:
        return len(_KERNEL_CACHE)


def generation() -> int:
    """Number of resets so far: a kernel obtained under another generation is stale."""
    return _generation


def reset_cache_for_tests() -> None:
    """Empty the cache and unload the native modules if the library is loaded."""
    from .. import _lib

    global _generation
    with _CACHE_LOCK:
        _KERNEL_CACHE.clear()
        _generation += 1
        lib = _lib.loaded()
        if lib is not None:
            lib.ta_cache_reset()
