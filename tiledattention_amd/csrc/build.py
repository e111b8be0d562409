"""Build recipe for the native parts: gfx950 code objects and the C-ABI library.

Outputs (into ``tiledattention_amd/lib/`` unless told otherwise):

* ``attn_fwd_m<TM>_n<TN>.hsaco`` for TM, TN in {64, 128}: each holds the 32 kernels of
  one tile shape (dtype x head dim x causal x tail x accumulation), compiled from
  ``attn_fwd.hip`` with ``hipcc --genco --offload-arch=gfx950``;
* ``attn_fwd_pp.hsaco``: the eight-wave kernels (dtype x head dim x causal x tail) that
  serve the (128, 64) tile shape with fp32 accumulation, from ``attn_fwd_pp.hip``;
* ``attn_fwd_wide.hsaco``: the short-row kernels (32 query rows a workgroup, the keys split
  across its eight waves) that serve 64-row tiles on small grids, from ``attn_fwd_wide.hip``;
* ``libtiledattn.so``: the host library implementing ``include/tiledattn.h``, linked from
  ``tiledattn.cpp`` (g++) and ``tiledattn_static.hip`` (hipcc; the static device scratch of
  ``ta_sdpa_fwd_split_static``);
* ``libtiledattn_torch.so``: the C++ torch operator ``tiledattention::sdpa_fwd``
  (``torch_ext.cpp``, g++ against the installed torch), linked to ``libtiledattn.so``.

Run as ``python -m tiledattention_amd.csrc.build``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
REPO = PKG.parent
LIB_DIR = PKG / "lib"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"
TILES = ((64, 64), (64, 128), (128, 64), (128, 128))

# Packed-fp32 VALU forms are kept out of every HIP build (see the kernel notes).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; a ROCm toolchain is required to build")
    return path


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}")


def code_object_cmd(tm: int, tn: int, out_dir: Path) -> list[str]:
    out = out_dir / f"attn_fwd_m{tm}_n{tn}.hsaco"
    return [
        _hipcc(),
        *HIP_FLAGS,
        "--genco",
        f"-DTA_TILE_M={tm}",
        f"-DTA_TILE_N={tn}",
        "-o",
        str(out),
        str(HERE / "attn_fwd.hip"),
    ]


def pp_code_object_cmd(out_dir: Path) -> list[str]:
    return [
        _hipcc(),
        *HIP_FLAGS,
        "--genco",
        "-o",
        str(out_dir / "attn_fwd_pp.hsaco"),
        str(HERE / "attn_fwd_pp.hip"),
    ]


def wide_code_object_cmd(out_dir: Path) -> list[str]:
    return [
        _hipcc(),
        *HIP_FLAGS,
        "--genco",
        "-o",
        str(out_dir / "attn_fwd_wide.hsaco"),
        str(HERE / "attn_fwd_wide.hip"),
    ]


def static_object_cmd(obj: Path) -> list[str]:
    """The library's HIP translation unit (a device array, no kernels) as a PIC object."""
    return [_hipcc(), *HIP_FLAGS, "-fPIC", "-Wall", "-c", "-o", str(obj), str(HERE / "tiledattn_static.hip")]


def library_cmd(out_dir: Path, static_obj: Path) -> list[str]:
    return [
        os.environ.get("CXX", "g++"),
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Wall",
        "-D__HIP_PLATFORM_AMD__",
        f"-I{ROCM / 'include'}",
        f"-I{REPO / 'include'}",
        "-o",
        str(out_dir / "libtiledattn.so"),
        str(HERE / "tiledattn.cpp"),
        str(static_obj),
        f"-L{ROCM / 'lib'}",
        f"-Wl,-rpath,{ROCM / 'lib'}",
        "-Wl,--no-undefined",
        "-lamdhip64",
        "-ldl",
    ]


def torch_ext_cmd(out_dir: Path) -> list[str]:
    """The C++ torch operator (torch.ops.tiledattention.sdpa_fwd) over the C ABI, linked
    against the installed torch and libtiledattn.so beside it."""
    import torch
    from torch.utils import cpp_extension

    tlib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(bool(getattr(torch._C, "_GLIBCXX_USE_CXX11_ABI", True)))
    return [
        os.environ.get("CXX", "g++"),
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Wall",
        "-D__HIP_PLATFORM_AMD__",
        "-DUSE_ROCM",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *[f"-I{p}" for p in cpp_extension.include_paths()],
        f"-I{ROCM / 'include'}",
        f"-I{REPO / 'include'}",
        "-o",
        str(out_dir / "libtiledattn_torch.so"),
        str(HERE / "torch_ext.cpp"),
        f"-L{tlib}",
        f"-Wl,-rpath,{tlib}",
        "-ltorch",
        "-ltorch_cpu",
        "-lc10",
        "-lc10_hip",
        "-ltorch_hip",
        f"-L{out_dir}",
        "-ltiledattn",
        "-Wl,-rpath,$ORIGIN",
        f"-L{ROCM / 'lib'}",
        f"-Wl,-rpath,{ROCM / 'lib'}",
        "-lamdhip64",
    ]


def _build_library(out_dir: Path) -> None:
    with tempfile.TemporaryDirectory(prefix="tiledattn_build_") as tmp:
        obj = Path(tmp) / "tiledattn_static.o"
        _run(static_object_cmd(obj))
        _run(library_cmd(out_dir, obj))
    _run(torch_ext_cmd(out_dir))


def build(out_dir: Path | None = None, jobs: int | None = None) -> Path:
    """Compile every code object and the host library; return the output directory."""
    out = Path(out_dir) if out_dir is not None else LIB_DIR
    out.mkdir(parents=True, exist_ok=True)
    cmds = [code_object_cmd(tm, tn, out) for tm, tn in TILES]
    cmds += [pp_code_object_cmd(out), wide_code_object_cmd(out)]
    workers = jobs or min(len(cmds) + 1, max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=workers) as pool:
        futs = [pool.submit(_run, c) for c in cmds] + [pool.submit(_build_library, out)]
        for fut in futs:
            fut.result()
    return out


if __name__ == "__main__":
    d = build()
    print(f"built into {d}")
    sys.exit(0)
