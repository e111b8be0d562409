"""Ported from the reference's tests/test_tiledattention.py:4-8, plus the callable-module fix."""

from __future__ import annotations


def test_tiledattention_exports_sdpa() -> None:
    import tiledattention

    assert hasattr(tiledattention, "sdpa")
    assert callable(tiledattention.sdpa)


def test_sdpa_stays_callable_after_submodule_import() -> None:
    # Importing the submodule rebinds the package attribute to the module object; the
    # module forwards calls, so the public name stays callable.
    import tiledattention
    import tiledattention.sdpa  # noqa: F401

    assert callable(tiledattention.sdpa)
    assert callable(tiledattention.sdpa.sdpa)


def test_public_names_match_reference() -> None:
    import tiledattention

    assert set(tiledattention.__all__) == {
        "__version__",
        "sdpa",
        "TiledAttentionError",
        "UnsupportedPlatformError",
        "InvalidShapeError",
        "DTypeNotSupportedError",
        "DependencyError",
    }
    for name in ("UnsupportedPlatformError", "InvalidShapeError", "DTypeNotSupportedError", "DependencyError"):
        assert issubclass(getattr(tiledattention, name), tiledattention.TiledAttentionError)


def test_reference_module_paths_import_in_a_fresh_interpreter() -> None:
    # The reference's callers import these names (benchmark-gb10/run_study.py:17-18,
    # run_reduced_optimization.py:10-11, tests/test_errors.py:7, tests/test_sdpa_shapes.py:8-12);
    # a fresh interpreter with only the checkout on sys.path must resolve all of them.
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    code = (
        "from tiledattention import sdpa\n"
        "import tiledattention._runtime as runtime\n"
        "from tiledattention._runtime import get_torch_module, _reset_runtime_cache_for_tests\n"
        "from tiledattention.kernels.compile_cache import reset_cache_for_tests, get_kernel\n"
        "from tiledattention.kernels.flash_fwd import run_flash_fwd\n"
        "from tiledattention.utils.checks import validate_sdpa_inputs\n"
        "from tiledattention._errors import InvalidShapeError, DTypeNotSupportedError\n"
        "import tiledattention.sdpa as sdpa_mod\n"
        "assert callable(sdpa) and callable(sdpa_mod.run_flash_fwd)\n"
        "print('ok')\n"
    )
    out = subprocess.run([sys.executable, "-c", code], cwd=str(root), capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "ok"


def test_native_package_alias_reexports_the_same_objects() -> None:
    import tiledattention
    import tiledattention_amd

    assert tiledattention_amd.__all__ == tiledattention.__all__
    for name in ("TiledAttentionError", "InvalidShapeError", "DependencyError", "__version__"):
        assert getattr(tiledattention_amd, name) is getattr(tiledattention, name)
    assert callable(tiledattention_amd.sdpa)
    assert (tiledattention_amd.CSRC_DIR / "tiledattn.cpp").exists()
    from tiledattention import _lib

    assert _lib.lib_dir() == tiledattention_amd.LIB_DIR
