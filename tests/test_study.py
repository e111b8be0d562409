"""The study harness on the CPU: the reference study's formulas, failure classification, file
schemas and the rocprofv3 summary (synthetic profiler output; nothing runs on a GPU)."""

from __future__ import annotations

import csv
import math

import pytest

from tiledattention import study


def test_bench_schema_is_the_reference_column_order():
    # run_study.py:610-629
    assert study.BENCH_FIELDS == (
        "method", "baseline_name", "dtype", "causal", "B", "H", "S", "D", "flops_forward", "median_ms",
        "p95_ms", "throughput_tokens_per_s", "tflops_per_s", "approx_bw_gbps", "status", "status_detail")
    assert study.TUNE_FIELDS[:3] == ("regime", "S", "D")


def test_formulas_closed_form():
    assert study.attention_forward_flops(b=1, h=8, s=8192, d=128, causal=False) == 4 * 8 * 8192**2 * 128
    assert study.attention_forward_flops(b=1, h=8, s=8192, d=128, causal=True) == 2 * 8 * 8192 * 8193 * 128
    assert study.throughput_tokens_per_s(b=2, h=4, s=100, median_ms=2.0) == 2 * 4 * 100 / 2e-3
    assert study.tflops_per_s(flops=3e12, median_ms=1000.0) == pytest.approx(3.0)
    assert study.approximate_bw_gbps(b=1, h=1, s=1000, d=64, bytes_per_elem=2, median_ms=1.0) == \
        pytest.approx(4 * 1000 * 64 * 2 / 1e-3 / 1e9)


def test_p95_matches_statistics_quantiles():
    vals = [float(x) for x in range(1, 21)]
    assert study.p95(vals) == pytest.approx(19.95)
    assert study.p95([3.0]) == 3.0
    with pytest.raises(ValueError):
        study.p95([])


@pytest.mark.parametrize("method,exc,status", [
    ("torch_sdpa_flash_forced", ValueError("bad"), "unsupported"),
    ("tiledattention", ValueError("bad"), "runtime_error"),
    ("flashattention", TypeError("x"), "unsupported"),
    ("tiledattention", RuntimeError("HIP out of memory. Tried"), "oom"),
    ("torch_sdpa_cudnn_forced", RuntimeError("No available kernel. Aborting execution."), "unsupported"),
    ("torch_sdpa", RuntimeError("No available kernel"), "runtime_error"),
    ("torch_sdpa_efficient_forced", RuntimeError("illegal memory access"), "runtime_error"),
    ("standard_eager", KeyError("k"), "runtime_error"),
    ("torch_sdpa_math", study.PlatformSkip("bf16 math path not run"), "unsupported"),
])
def test_failure_classification(method, exc, status):
    got, detail = study.classify_failure(method, exc)
    assert got == status
    assert detail and len(detail) <= 220


def _row(method, med, s=512, status="ok"):
    return {"method": method, "baseline_name": "torch_sdpa", "dtype": "bfloat16", "causal": True, "B": 1, "H": 8,
            "S": s, "D": 128, "flops_forward": 1.0, "median_ms": med, "p95_ms": med, "throughput_tokens_per_s": 1.0,
            "tflops_per_s": 2.0, "approx_bw_gbps": 3.0, "status": status, "status_detail": ""}


def test_csv_and_summary(tmp_path):
    rows = [_row("tiledattention", 0.5), _row("torch_sdpa", 2.0), _row("torch_sdpa_math", math.nan, status="unsupported")]
    study.write_csv(tmp_path / "b.csv", rows, study.BENCH_FIELDS)
    got = list(csv.DictReader((tmp_path / "b.csv").open()))
    assert list(got[0].keys()) == list(study.BENCH_FIELDS)
    assert got[2]["median_ms"] == "nan" and got[2]["status"] == "unsupported"
    tune = [{"regime": "Short S", "S": 1024, "D": 128, "best_TM": 128, "best_TN": 64, "best_median_ms": 1.0,
             "runner_TM": 64, "runner_TN": 64, "runner_median_ms": 1.25, "sensitivity_drop_percent": 25.0}]
    study.write_summary(tmp_path / "s.md", rows, tune)
    text = (tmp_path / "s.md").read_text()
    assert "| bfloat16 | True | 512 | 128 | 0.500 | 2.000 | 2.000 | 4.000 | ok |" in text
    assert "(128, 64)" in text and "25.000" in text
    with pytest.raises(ValueError):
        study.write_csv(tmp_path / "e.csv", [], study.BENCH_FIELDS)


def _write(path, header, rows):
    with path.open("w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_rocprof_summary_from_profiler_csvs(tmp_path):
    d = tmp_path / "prof"
    (d / "pass1").mkdir(parents=True)
    _write(d / "run_kernel_stats.csv", ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs",
                                        "MaxNs", "StdDev"],
           [["ta_fwd_pp_bf16_d128_c1_t0", 10, 1276340, 127634.0, 99.9, 1, 2, 3], ["other", 1, 5, 5.0, 0.1, 1, 1, 0]])
    hdr = ["Correlation_Id", "Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    rows = []
    for disp in (1, 2):
        rows += [[disp, disp, "ta_fwd_pp_bf16_d128_c1_t0", "SQ_VALU_MFMA_BUSY_CYCLES", 69206016.0],
                 [disp, disp, "ta_fwd_pp_bf16_d128_c1_t0", "SQ_VALU_MFMA_BUSY_CYCLES", 69206016.0],  # 2 dims
                 [disp, disp, "ta_fwd_pp_bf16_d128_c1_t0", "GRBM_GUI_ACTIVE", 2016856.0],
                 [disp, disp, "ta_fwd_pp_bf16_d128_c1_t0", "SQ_LDS_BANK_CONFLICT", 0.0],
                 [disp, disp, "copy", "GRBM_GUI_ACTIVE", 5.0]]
    _write(d / "pass1" / "run_counter_collection.csv", hdr, rows)
    m = study.rocprof_metrics(d, "ta_fwd")
    assert m["kernel"] == "ta_fwd_pp_bf16_d128_c1_t0"
    assert m["kernel_ms"] == pytest.approx(0.127634)
    assert m["SQ_VALU_MFMA_BUSY_CYCLES"] == pytest.approx(138412032.0)
    assert study.mfma_busy_pct(m) == pytest.approx(100 * 138412032.0 / (2016856.0 / 8 * 1024))
    study.write_rocprof_summary(tmp_path / "r.md", [("tiledattention", m)], {"Shape": "B=1 H=8 S=8192 D=128"})
    text = (tmp_path / "r.md").read_text()
    assert "# rocprofv3 One-Pass Summary" in text and "`ta_fwd_pp_bf16_d128_c1_t0`" in text
    assert "| tiledattention | `ta_fwd_pp_bf16_d128_c1_t0` | 0.128 | 53.6" in text
    assert "| tiledattention | GRBM_GUI_ACTIVE | 2016856.000 |" in text  # every counter's mean
    assert study.main(["--out", str(tmp_path / "o"), "--rocprof-dir", str(d)]) == 0
    assert (tmp_path / "o" / "rocprof_summary.md").exists()


def test_kernel_trace_table_per_kernel_and_grid(tmp_path):
    """Dispatch durations grouped by (kernel, workgroups = Grid_Size_X / Workgroup_Size_X):
    one symbol at two grid sizes is two rows; other kernels are filtered out."""
    d = tmp_path / "kt"
    d.mkdir()
    hdr = ["Kernel_Name", "Grid_Size_X", "Workgroup_Size_X", "Start_Timestamp", "End_Timestamp"]
    rows = [["ta_fwd_pp64_bf16_d128_c1_t0", 64 * 512, 512, 1000, 9800],      # 8.8 us
            ["ta_fwd_pp64_bf16_d128_c1_t0", 64 * 512, 512, 20000, 28600],    # 8.6 us
            ["ta_fwd_pp64_bf16_d128_c1_t0", 64 * 512, 512, 30000, 39000],    # 9.0 us
            ["ta_fwd_pp64_bf16_d128_c1_t0", 128 * 512, 512, 50000, 61760],   # 11.76 us
            ["copy_kernel", 1024, 256, 0, 100]]
    _write(d / "run_kernel_trace.csv", hdr, rows)
    t = study.kernel_trace_table(d, "ta_fwd")
    assert [(r["kernel"], r["workgroups"], r["calls"]) for r in t] == [
        ("ta_fwd_pp64_bf16_d128_c1_t0", 64, 3), ("ta_fwd_pp64_bf16_d128_c1_t0", 128, 1)]
    assert t[0]["median_us"] == pytest.approx(8.8) and t[0]["min_us"] == pytest.approx(8.6)
    assert t[0]["mean_us"] == pytest.approx((8.8 + 8.6 + 9.0) / 3)
    assert study.main(["--out", str(tmp_path / "o"), "--rocprof-dir", str(d), "--trace-table"]) == 0
    text = (tmp_path / "o" / "kernel_trace.md").read_text()
    assert "| ta_fwd_pp64_bf16_d128_c1_t0 | 128 | 1 | 11.76 | 11.76 | 11.76 |" in text


def test_diagnose_flags():
    assert any("underfed" in x for x in study.diagnose({"SQ_VALU_MFMA_BUSY_CYCLES": 10.0, "GRBM_GUI_ACTIVE": 8.0 * 1.0}))
    assert any("bank conflicts" in x for x in study.diagnose({"SQ_LDS_BANK_CONFLICT": 5.0}))
    assert study.diagnose({}) == ["No single dominant bottleneck from coarse counters; see the kernel trace."]
