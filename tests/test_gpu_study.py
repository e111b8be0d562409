"""The study harness on the GPU: a tiny grid through every method, the tuning sweep and the
CLI's files (schemas and statuses), and every timed method's output against the oracle."""

from __future__ import annotations

import csv
import math

import pytest

from tests.parity_util import say
from tiledattention import study

pytestmark = pytest.mark.gpu

OK_OR_SKIPPED = {"ok", "unsupported", "runtime_error"}


def test_tiny_grid_every_method(gpu):
    say("study: run_benchmark B1 H2 S128 D{64,160} fp16/bf16 causal/non-causal, warmup 1 iters 2")
    rows = study.run_benchmark(b=1, h=2, s_values=[128], d_values=[64, 160], dtypes=["float16", "bfloat16"],
                               causal_flags=[False, True], warmup=1, iters=2)
    methods = {r["method"] for r in rows}
    assert {"tiledattention", "torch_sdpa", "torch_sdpa_math", "standard_eager"} <= methods
    assert set(study.FORCED_METHODS) <= methods
    for r in rows:
        assert tuple(r.keys()) == study.BENCH_FIELDS
        assert r["status"] in OK_OR_SKIPPED, r
        if r["status"] != "ok":
            assert math.isnan(r["median_ms"]) and r["status_detail"]
    ours = [r for r in rows if r["method"] == "tiledattention"]
    assert len(ours) == 8 and all(r["status"] == "ok" and r["median_ms"] > 0 for r in ours)
    for r in rows:
        if r["method"] == "standard_eager":
            assert r["status"] == "ok"
        if r["method"] == "torch_sdpa_math" and r["dtype"] == "bfloat16":
            assert r["status"] == "unsupported"


def test_tune_and_cli_files(gpu, tmp_path):
    say("study: run_tune at S=256 over the reference's candidate tiles")
    rows = study.run_tune(b=1, h=2, warmup=1, iters=2, regimes=(("Short S", 256),))
    assert len(rows) == 1 and tuple(rows[0].keys()) == study.TUNE_FIELDS
    assert (rows[0]["best_TM"], rows[0]["best_TN"]) in {(64, 64), (64, 128), (128, 64), (128, 128)}
    say("study: CLI on a tiny grid")
    rc = study.main(["--out", str(tmp_path), "--seqs", "128", "--dims", "64", "--dtypes", "float16",
                     "--warmup", "1", "--iters", "2", "--no-tune", "--heads", "2"])
    assert rc == 0
    got = list(csv.DictReader((tmp_path / "benchmark_results.csv").open()))
    assert list(got[0].keys()) == list(study.BENCH_FIELDS)
    assert (tmp_path / "table3_reproducibility.md").read_text().startswith("# Table 3")
    assert "| float16 | False | 128 | 64 |" in (tmp_path / "study_summary.md").read_text()


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_harness_methods_compute_attention(gpu, dtype, causal):
    """Every method the study times computes the attention it is timed for: the inputs the
    harness generates (torch.manual_seed(1234), N(0,1) on the GPU, run_study.py:526-529),
    each method's output against the explicit fp32 oracle on the same values.  The
    ``tiledattention`` rows meet the north-star bound; PyTorch's own paths 5e-2 (the eager
    path rounds its scores to the input dtype; the check is that they are attention, which
    a transposed operand, a dropped scale or a shifted mask would miss by far more)."""
    import torch

    from tests.parity_util import TOL, check_close, oracle_f32

    b, h, s, d = 1, 2, 200, 64
    torch.manual_seed(1234)
    q = torch.randn((b, h, s, d), device="cuda", dtype=getattr(torch, dtype))
    k = torch.randn((b, h, s, d), device="cuda", dtype=getattr(torch, dtype))
    v = torch.randn((b, h, s, d), device="cuda", dtype=getattr(torch, dtype))
    ref = oracle_f32(q.cpu(), k.cpu(), v.cpu(), causal=causal)
    checked = set()
    for method, fn in study.build_methods(q, k, v, causal=causal, forced_backends=True, flashattention=True):
        say(f"study method {method} {dtype} causal={causal} (1,2,200,64)")
        try:
            out = fn()
        except Exception as exc:  # the harness classifies these; only ok methods are checked
            status, _ = study.classify_failure(method, exc)
            assert status in OK_OR_SKIPPED and method != "tiledattention", (method, exc)
            continue
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        tol = TOL[dtype] if method == "tiledattention" else 5e-2
        check_close(got, ref, dtype, tol=tol, what=f"study {method}")
        checked.add(method)
    assert {"tiledattention", "standard_eager"} <= checked
