"""Ported from the reference's tests/test_tiledattention.py:4-8, plus the callable-module fix."""

from __future__ import annotations


def test_tiledattention_exports_sdpa() -> None:
    import tiledattention_amd

    assert hasattr(tiledattention_amd, "sdpa")
    assert callable(tiledattention_amd.sdpa)


def test_sdpa_stays_callable_after_submodule_import() -> None:
    # Importing the submodule rebinds the package attribute to the module object; the
    # module forwards calls, so the public name stays callable.
    import tiledattention_amd
    import tiledattention_amd.sdpa  # noqa: F401

    assert callable(tiledattention_amd.sdpa)
    assert callable(tiledattention_amd.sdpa.sdpa)


def test_public_names_match_reference() -> None:
    import tiledattention_amd

    assert set(tiledattention_amd.__all__) == {
        "__version__",
        "sdpa",
        "TiledAttentionError",
        "UnsupportedPlatformError",
        "InvalidShapeError",
        "DTypeNotSupportedError",
        "DependencyError",
    }
    for name in ("UnsupportedPlatformError", "InvalidShapeError", "DTypeNotSupportedError", "DependencyError"):
        assert issubclass(getattr(tiledattention_amd, name), tiledattention_amd.TiledAttentionError)
