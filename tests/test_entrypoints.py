"""Driver-facing entry points on the CPU: bench.py's one-GPU contract, __graft_entry__."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=60)
    assert proc.returncode == 2
    assert "one GPU only" in proc.stderr
    assert proc.stdout == ""


def test_graft_entry_exposes_build_and_smoke():
    import importlib

    sys.path.insert(0, str(ROOT))
    mod = importlib.import_module("__graft_entry__")
    assert callable(mod.build) and callable(mod.smoke)
