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


def test_bench_workload_inputs_and_counts_match_the_oracle_helpers():
    """bench.py generates its inputs and counts work on its own (the product and the bench
    never import the oracle outside the CPU-baseline leg); both must equal what the parity
    tests feed the oracle, so every timed configuration is one the tests check."""
    import torch

    sys.path.insert(0, str(ROOT))
    import bench
    from oracle import oracle as O

    for kw in ({}, {"scale_inputs": 0.5}, {"outlier_frac": 0.01, "outlier_gain": 20.0, "outlier_seed": 1235}):
        for dtype in ("float16", "bfloat16"):
            a = bench.make_inputs((1, 2, 64, 64), dtype, 1234, **kw)
            b = O.make_inputs((1, 2, 64, 64), dtype, 1234, **kw)
            for x, y in zip(a, b):
                assert x.dtype == y.dtype and torch.equal(x, y)
    for causal in (False, True):
        assert bench.flops_of(1, 8, 8192, 128, causal) == O.attention_forward_flops(b=1, h=8, s=8192, d=128,
                                                                                    causal=causal)
    assert bench.alg_bytes(1, 8, 8192, 128) == O.approximate_bytes(b=1, h=8, s=8192, d=128, bytes_per_elem=2)
    vals = [0.1 * i for i in range(1, 60)]
    assert bench.p95(vals) == O.p95(vals)
    assert bench.flops_of(1, 8, 8192, 128, True) == 137438953472.0  # 2*B*H*S^2*D


def test_bench_mantissa_clearing_keeps_sign_and_exponent():
    """The ceiling block's operands: every value keeps its sign and exponent and only the
    top ``keep_bits`` mantissa bits; bf16 with none kept is +-2^e exactly (truncation
    toward zero, |x'| <= |x| < 2|x'|)."""
    import torch

    sys.path.insert(0, str(ROOT))
    import bench

    g = torch.Generator().manual_seed(5)
    x = torch.randn(4096, generator=g)
    for dtype, man in ((torch.bfloat16, 7), (torch.float16, 10)):
        t = x.to(dtype)
        for keep in (0, 3):
            y = bench.clear_mantissa(t, keep)
            assert y.dtype == dtype
            tb = t.view(torch.int16).to(torch.int32) & 0xFFFF
            yb = y.view(torch.int16).to(torch.int32) & 0xFFFF
            low = (1 << (man - keep)) - 1
            assert torch.equal(yb & low, torch.zeros_like(yb))
            assert torch.equal(yb, tb & (0xFFFF ^ low))
            tf, yf = t.float().abs(), y.float().abs()
            nz = tf > 0
            assert (yf <= tf).all() and (tf[nz] < 2 * yf[nz]).all()
            assert torch.equal(torch.sign(t.float()), torch.sign(y.float()))
        y0 = bench.clear_mantissa(t, 0).float().abs()
        nz = y0 > 0
        assert torch.equal(torch.exp2(torch.log2(y0[nz]).round()), y0[nz])  # powers of two


def test_bench_reference_grid_covers_the_metric():
    """The grid block's reference points: every (dtype, causal, S, D) of the metric at the
    reference's B1 H8 grid, the headline point equal to the line the bench compares with."""
    sys.path.insert(0, str(ROOT))
    import bench

    keys = {(dt, c, s, d) for dt in ("float16", "bfloat16") for c in (False, True)
            for s in bench.GRID_S for d in (64, 128)}
    assert set(bench.REFERENCE_GB10_GRID) == keys
    line_no, ref = bench.REFERENCE_GB10_GRID[("bfloat16", True, 8192, 128)]
    assert line_no == 548 and abs(ref - bench.REFERENCE_GB10_C3_S8192) < 0.01
    lines = [v[0] for v in bench.REFERENCE_GB10_GRID.values()]
    assert len(set(lines)) == len(lines)


def test_bench_small_block_stays_in_the_planned_range():
    """The small-grid block's shapes are ones whose 64-row blocks fill at most half of an
    MI355X's 256 CUs (where the 64-row split is planned), and its alternatives name knobs
    the library reads."""
    sys.path.insert(0, str(ROOT))
    import bench
    from tiledattention.kernels import flash_fwd

    for bh, s in bench.SMALL_GRIDS:
        assert 2 * bh * -(-s // 64) <= 256, (bh, s)
    names = {"TILEDATTN_" + k.upper() for _, env in bench.SMALL_ALTERNATIVES for k in env}
    assert names <= set(flash_fwd._KNOBS)
