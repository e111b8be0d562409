"""The study harness on the GPU: a tiny grid through every method, the tuning sweep and the
CLI's files (schemas and statuses; the timings themselves are not checked)."""

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
