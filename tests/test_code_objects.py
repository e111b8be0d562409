"""Code-object metadata of the built kernels: no kernel spills registers to scratch.

Reads the AMDGPU metadata notes of every `tiledattention_amd/lib/*.hsaco` (unbundled with
clang-offload-bundler, printed with llvm-readelf): for each kernel `.vgpr_spill_count`,
`.sgpr_spill_count` and `.private_segment_fixed_size` must be 0.  Skipped when the ROCm LLVM
tools or the built code objects are absent.
"""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "tiledattention_amd" / "lib"
LLVM = Path("/opt/rocm/llvm/bin")


def _tool(name: str) -> str | None:
    p = LLVM / name
    return str(p) if p.exists() else shutil.which(name)


def _kernels(hsaco: Path, tmp: Path) -> list[dict[str, str]]:
    bundler, readelf = _tool("clang-offload-bundler"), _tool("llvm-readelf")
    elf = tmp / (hsaco.stem + ".elf")
    r = subprocess.run([bundler, "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                        f"--input={hsaco}", f"--output={elf}", "--unbundle"], capture_output=True)
    if r.returncode != 0:  # not a bundle: the file is the ELF itself
        elf = hsaco
    notes = subprocess.run([readelf, "--notes", str(elf)], capture_output=True, text=True, check=True).stdout
    out = []
    for block in re.split(r"\n\s+- \.agpr_count", notes)[1:]:
        fields = dict(re.findall(r"\.([a-z_]+):\s+(\S+)", block))
        out.append(fields)
    return out


def test_no_kernel_spills_to_scratch(tmp_path):
    if _tool("clang-offload-bundler") is None or _tool("llvm-readelf") is None:
        pytest.skip("ROCm LLVM tools not found")
    objs = sorted(LIB.glob("*.hsaco"))
    if not objs:
        pytest.skip("code objects not built")
    seen = 0
    bad = []
    for h in objs:
        for k in _kernels(h, tmp_path):
            seen += 1
            spills = (int(k.get("vgpr_spill_count", 0)), int(k.get("sgpr_spill_count", 0)),
                      int(k.get("private_segment_fixed_size", 0)))
            if any(spills):
                bad.append((h.name, k.get("name"), spills))
    assert seen > 100, f"only {seen} kernels found in {LIB}"
    assert not bad, f"kernels with spills / scratch (vgpr, sgpr, private bytes): {bad}"
