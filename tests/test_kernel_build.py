"""Kernel-package layout (tiledattention_amd.kernel_build): the ``build/<variant>/tiledattention``
tree that the reference's ``example.py:15`` loads with ``kernels.get_local_kernel``, written
from the built library and code objects, and loaded by the same resolution rule."""
from __future__ import annotations

import ctypes
import re

import pytest

from tiledattention import _lib

kb = pytest.importorskip("tiledattention_amd.kernel_build")


@pytest.fixture(scope="module")
def package(tmp_path_factory):
    if not (kb.LIB_SRC / "libtiledattn.so").exists():
        pytest.skip("native library not built")
    root = tmp_path_factory.mktemp("kbuild")
    return root, kb.write_kernel_package(root / "build")


def test_variant_name():
    import torch

    v = kb.build_variant()
    assert re.fullmatch(r"torch\d+-cxx(11|98)-rocm\d+-[a-z0-9_]+-linux", v), v
    major, minor = torch.__version__.split("+")[0].split(".")[:2]
    assert v.startswith(f"torch{major}{minor}-")


def test_layout_mirrors_the_package(package):
    root, pkg = package
    assert pkg == root / "build" / kb.build_variant() / "tiledattention"
    src = {p.relative_to(kb.PY_SRC) for p in kb.PY_SRC.rglob("*.py") if "__pycache__" not in p.parts}
    got = {p.relative_to(pkg) for p in pkg.rglob("*.py")}
    assert got == src | {kb.Path("_ops.py")}
    assert (pkg / "lib" / "libtiledattn.so").exists()
    assert {p.name for p in (pkg / "lib").glob("*.hsaco")} == {p.name for p in kb.LIB_SRC.glob("*.hsaco")}
    # rewriting replaces the tree
    again = kb.write_kernel_package(root / "build")
    assert again == pkg and (pkg / "_ops.py").exists()


def test_local_loader_imports_a_separate_module(package):
    import tiledattention

    root, pkg = package
    kernel = kb.load_local_kernel(root)  # resolves <root>/build/<variant>/tiledattention
    assert kernel is not tiledattention and kernel.__name__.startswith("tiledattention_")
    assert kb.load_local_kernel(root) is kernel
    assert callable(kernel.sdpa) and set(kernel.__all__) == set(tiledattention.__all__)
    import importlib

    assert importlib.import_module(f"{kernel.__name__}._lib").lib_dir() == pkg / "lib"
    ops = importlib.import_module(f"{kernel.__name__}._ops")
    assert ops.add_op_namespace_prefix("sdpa_fwd") == "tiledattention::sdpa_fwd"
    # the package's own copy of the C-ABI library loads and reports this ABI
    lib = ctypes.CDLL(str(pkg / "lib" / "libtiledattn.so"))
    lib.ta_abi_version.restype = ctypes.c_int
    assert lib.ta_abi_version() == _lib.ABI_VERSION
    with pytest.raises(FileNotFoundError):
        kb.load_local_kernel(root / "nowhere")
