"""Runtime-gate errors, re-targeted from the reference's tests/test_errors.py:35-100.

Reference check -> here: "requires CUDA + Blackwell GPU" -> "requires a ROCm (HIP) GPU";
"compute capability 9.0" -> "architecture gfx942"; "CuPy is required" / "cuTile ... could
not be imported" -> the native library or its code objects missing.  Same exception types.
"""

from __future__ import annotations

import pytest

from tests.fakes import make_torch_module
from tiledattention._errors import DependencyError, UnsupportedPlatformError
from tiledattention._runtime import _reset_runtime_cache_for_tests, require_supported_runtime


def _raise_dependency_error(message: str) -> None:
    raise DependencyError(message)


def test_runtime_raises_on_gpu_unavailable(monkeypatch: pytest.MonkeyPatch) -> None:
    import tiledattention._runtime as runtime

    monkeypatch.setattr(runtime, "_get_torch_module", lambda: make_torch_module(cuda_available=False))
    _reset_runtime_cache_for_tests()
    with pytest.raises(UnsupportedPlatformError, match=r"requires a ROCm \(HIP\) GPU"):
        require_supported_runtime()


def test_runtime_raises_on_non_rocm_torch(monkeypatch: pytest.MonkeyPatch) -> None:
    import tiledattention._runtime as runtime

    monkeypatch.setattr(runtime, "_get_torch_module",
                        lambda: make_torch_module(cuda_available=True, hip=None))
    _reset_runtime_cache_for_tests()
    with pytest.raises(UnsupportedPlatformError, match="built for ROCm"):
        require_supported_runtime()


def test_runtime_raises_on_non_gfx950_gpu(monkeypatch: pytest.MonkeyPatch) -> None:
    import tiledattention._runtime as runtime

    monkeypatch.setattr(runtime, "_get_torch_module",
                        lambda: make_torch_module(cuda_available=True, arch="gfx942:sramecc+:xnack-"))
    _reset_runtime_cache_for_tests()
    with pytest.raises(UnsupportedPlatformError, match="architecture gfx942"):
        require_supported_runtime()


def test_runtime_raises_on_missing_native_library(monkeypatch: pytest.MonkeyPatch) -> None:
    import tiledattention._runtime as runtime

    monkeypatch.setattr(runtime, "_get_torch_module", lambda: make_torch_module(cuda_available=True))
    monkeypatch.setattr(runtime, "_get_native_library",
                        lambda: _raise_dependency_error("Native library libtiledattn.so is missing."))
    _reset_runtime_cache_for_tests()
    with pytest.raises(DependencyError, match="Native library"):
        require_supported_runtime()


def test_missing_library_file_is_a_dependency_error(monkeypatch: pytest.MonkeyPatch, tmp_path) -> None:
    # The real loader, pointed at an empty directory: fails loudly, no fallback.
    from tiledattention import _lib

    monkeypatch.setenv("TILEDATTN_LIB_DIR", str(tmp_path))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(DependencyError, match="is missing"):
        _lib.load()


def test_missing_code_object_is_a_dependency_error(monkeypatch: pytest.MonkeyPatch, tmp_path) -> None:
    from tiledattention import _lib

    real = _lib.library_path()
    if not real.exists():
        pytest.skip("native library not built")
    (tmp_path / "libtiledattn.so").symlink_to(real)
    monkeypatch.setenv("TILEDATTN_LIB_DIR", str(tmp_path))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(DependencyError, match="code objects are missing"):
        _lib.load()


def test_gate_passes_with_fakes_and_is_cached(monkeypatch: pytest.MonkeyPatch) -> None:
    import tiledattention._runtime as runtime

    calls = []
    monkeypatch.setattr(runtime, "_get_torch_module", lambda: make_torch_module(cuda_available=True))
    monkeypatch.setattr(runtime, "_get_native_library", lambda: calls.append(1) or object())
    _reset_runtime_cache_for_tests()
    require_supported_runtime()
    require_supported_runtime()
    assert calls == [1]
    _reset_runtime_cache_for_tests()
