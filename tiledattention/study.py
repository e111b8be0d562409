"""Study harness: times the forward against PyTorch's attention paths and writes the
reference study's result files.

Restates the reference's study pipeline (``benchmark-gb10/run_study.py``) for this build:

* ``benchmark_results.csv`` with the reference's columns and order (``run_study.py:610-629``):
  method, baseline_name, dtype, causal, B, H, S, D, flops_forward, median_ms, p95_ms,
  throughput_tokens_per_s, tflops_per_s, approx_bw_gbps, status, status_detail;
* the same methods (``:536-589``): ``tiledattention`` (this package), ``torch_sdpa``,
  ``torch_sdpa_math``, ``standard_eager``, the forced ``torch_sdpa_{flash,efficient,cudnn}``
  backends and ``flashattention`` when the ``flash_attn`` package imports;
* the same failure classification into ``unsupported`` / ``oom`` / ``runtime_error`` with
  NaN metrics (``:338-395``);
* ``tuning_results.csv`` (``:1230-1342``): best and runner-up (TILE_M, TILE_N) per regime;
* ``table3_reproducibility.md`` (``:398-480``) and ``study_summary.md``;
* ``rocprof_summary.md`` from a ``rocprofv3`` run, in the shape of the reference's Nsight
  one-pass summary (``run_ncu_profile.py:469-520``), via ``write_rocprof_summary``.

Differences, all recorded in ``status_detail`` where they apply: FLOPs are counted as the
reference study does (``2·B·H·S·(S+1)·D`` causal, ``:95-112``); inputs are seeded
``torch.manual_seed(1234)`` N(0,1) on the GPU as there (``:526-529``).  The bf16 math path
of ``torch_sdpa_math`` is not run, and ``torch_sdpa`` in bf16 is limited to the fused
backends (flash, efficient): PyTorch's bf16 math path calls batched products
(``torch.bmm``) whose right operand is a transposed view, a form known to fault MI355X GPUs
of the pool these measurements run on (a platform notice; it was never run here, so no run
of this build has shown the fault).  The eager baseline makes Kᵀ contiguous for the same
reason.  No figures are drawn (matplotlib is not a dependency).

Run: ``python -m tiledattention.study --out DIR [--seqs ...] [--dims ...]``.
"""

from __future__ import annotations

import argparse
import csv
import math
import os
import platform
import statistics
import subprocess
import sys
from pathlib import Path
from typing import Callable, Iterable

BENCH_FIELDS = (
    "method", "baseline_name", "dtype", "causal", "B", "H", "S", "D", "flops_forward",
    "median_ms", "p95_ms", "throughput_tokens_per_s", "tflops_per_s", "approx_bw_gbps",
    "status", "status_detail",
)
TUNE_FIELDS = (
    "regime", "S", "D", "best_TM", "best_TN", "best_median_ms", "runner_TM", "runner_TN",
    "runner_median_ms", "sensitivity_drop_percent",
)
BASELINE_NAME = "torch_sdpa"
# The reference's candidate tiles and regimes (run_study.py:1254-1255); tiles outside this
# build's {64, 128} x {64, 128} are measured as unsupported.
TUNE_CANDIDATES = ((32, 64), (64, 64), (64, 128), (64, 256), (128, 64), (128, 128), (128, 256))
TUNE_REGIMES = (("Short S", 1024), ("Mid S", 4096), ("Long S", 8192))
FORCED_METHODS = ("torch_sdpa_flash_forced", "torch_sdpa_efficient_forced", "torch_sdpa_cudnn_forced")

_UNSUPPORTED_PATTERNS = (
    "no viable backend",
    "no available kernel",
    "no execution plans support",
    "not supported",
    "not implemented",
    "does not support",
    "unable to find an engine",
)


# ---------------------------------------------------------------- metrics (run_study.py:30-150)

def p95(values: list[float]) -> float:
    """95th percentile as the reference computes it: the 19th of 20 quantiles."""
    if not values:
        raise ValueError("values must not be empty")
    if len(values) == 1:
        return values[0]
    return statistics.quantiles(values, n=20)[18]


def attention_forward_flops(*, b: int, h: int, s: int, d: int, causal: bool) -> float:
    """The study's FLOP count: 4·B·H·S²·D, causal 2·B·H·S·(S+1)·D."""
    if causal:
        return 2.0 * b * h * s * (s + 1) * d
    return 4.0 * b * h * s * s * d


def throughput_tokens_per_s(*, b: int, h: int, s: int, median_ms: float) -> float:
    return (b * h * s) / (median_ms / 1000.0)


def tflops_per_s(*, flops: float, median_ms: float) -> float:
    return flops / (median_ms / 1000.0) / 1e12


def approximate_bw_gbps(*, b: int, h: int, s: int, d: int, bytes_per_elem: int, median_ms: float) -> float:
    """q, k, v read and o written once."""
    return 4.0 * b * h * s * d * bytes_per_elem / (median_ms / 1000.0) / 1e9


# ---------------------------------------------------------------- failure classification

def _short(exc: BaseException) -> str:
    text = " ".join(str(exc).strip().split())
    return (text or exc.__class__.__name__)[:220]


class PlatformSkip(ValueError):
    """A method this platform does not run for a case: always ``unsupported``."""


def classify_failure(method: str, exc: BaseException) -> tuple[str, str]:
    """(status, detail) for a method that raised (run_study.py:371-395): TypeError/ValueError
    are ``unsupported`` for the optional backends and ``runtime_error`` otherwise; a
    RuntimeError mentioning out-of-memory is ``oom``; an optional backend's RuntimeError that
    reads like "no kernel for this case" is ``unsupported``; anything else is
    ``runtime_error``."""
    optional = method == "flashattention" or (method.startswith("torch_sdpa_") and method.endswith("_forced"))
    detail = _short(exc)
    if isinstance(exc, PlatformSkip):
        return "unsupported", detail
    if isinstance(exc, (TypeError, ValueError)):
        return ("unsupported" if optional else "runtime_error"), detail
    if isinstance(exc, RuntimeError):
        msg = str(exc).lower()
        if "out of memory" in msg:
            return "oom", detail
        if optional and any(p in msg for p in _UNSUPPORTED_PATTERNS):
            return "unsupported", detail
    return "runtime_error", detail


# ---------------------------------------------------------------- timing

def time_callable(fn: Callable[[], object], *, warmup: int, iters: int) -> tuple[float, float]:
    """Median and p95 of per-call GPU-event times, after ``warmup`` calls (run_study.py:48-75)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(iters):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        end.record()
        end.synchronize()
        times.append(float(start.elapsed_time(end)))
    return statistics.median(times), p95(times)


def time_method(method: str, fn: Callable[[], object], *, warmup: int, iters: int) -> tuple[float, float, str, str]:
    """(median_ms, p95_ms, status, detail); NaN metrics when the method fails."""
    import torch

    try:
        med, tail = time_callable(fn, warmup=warmup, iters=iters)
        return med, tail, "ok", ""
    except Exception as exc:  # classified below, as the reference does
        status, detail = classify_failure(method, exc)
        if status == "oom":
            torch.cuda.empty_cache()
        print(f"[study] warning: {method}: {status} ({detail}); writing NaN metrics", flush=True)
        return math.nan, math.nan, status, detail


# ---------------------------------------------------------------- methods

def standard_eager_attention(q, k, v, *, causal: bool, causal_mask=None):
    """softmax(q kᵀ / sqrt(D) with future keys at the dtype's minimum) v, softmax in fp32
    (run_study.py:304-335).  Kᵀ is made contiguous before the batched product."""
    import torch

    scale = 1.0 / math.sqrt(float(q.shape[-1]))
    scores = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
    if causal:
        if causal_mask is None:
            s = scores.shape[-1]
            causal_mask = torch.ones((1, 1, s, s), device=scores.device, dtype=torch.bool).triu(1)
        low = torch.tensor(torch.finfo(scores.dtype).min, dtype=scores.dtype, device=scores.device)
        scores = torch.where(causal_mask, low, scores)
    probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.matmul(probs, v)


def _sdpa_with(backends, q, k, v, causal: bool):
    import torch
    from torch.nn.attention import sdpa_kernel

    with sdpa_kernel(backends):
        return torch.nn.functional.scaled_dot_product_attention(q, k, v, dropout_p=0.0, is_causal=causal)


def _flash_attn_func():
    try:
        from flash_attn import flash_attn_func  # type: ignore[import-not-found]
    except Exception:
        return None
    return flash_attn_func


def build_methods(q, k, v, *, causal: bool, forced_backends: bool = True,
                  flashattention: bool = True) -> list[tuple[str, Callable[[], object]]]:
    """The study's methods for one case, in the reference's order."""
    import torch
    from torch.nn.attention import SDPBackend

    from . import sdpa

    bf16 = q.dtype == torch.bfloat16
    fused = [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]
    mask = torch.ones((1, 1, q.shape[2], q.shape[2]), device=q.device, dtype=torch.bool).triu(1) if causal else None

    def torch_sdpa():
        if bf16:
            return _sdpa_with(fused, q, k, v, causal)
        return torch.nn.functional.scaled_dot_product_attention(q, k, v, dropout_p=0.0, is_causal=causal)

    def torch_sdpa_math():
        if bf16:
            raise PlatformSkip("bf16 math path not run on this platform (batched product with a transposed operand)")
        return _sdpa_with([SDPBackend.MATH], q, k, v, causal)

    methods = [
        ("tiledattention", lambda: sdpa(q, k, v, causal=causal)),
        (BASELINE_NAME, torch_sdpa),
        ("torch_sdpa_math", torch_sdpa_math),
        ("standard_eager", lambda: standard_eager_attention(q, k, v, causal=causal, causal_mask=mask)),
    ]
    if forced_backends:
        for name, backend in zip(FORCED_METHODS, (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION,
                                                  SDPBackend.CUDNN_ATTENTION)):
            methods.append((name, lambda backend=backend: _sdpa_with([backend], q, k, v, causal)))
    fa = _flash_attn_func() if flashattention else None
    if fa is not None:
        methods.append(("flashattention",
                        lambda: fa(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), causal=causal)))
    return methods


# ---------------------------------------------------------------- benchmark and tuning

def run_benchmark(*, b: int, h: int, s_values: Iterable[int], d_values: Iterable[int],
                  dtypes: Iterable[str], causal_flags: Iterable[bool], warmup: int, iters: int,
                  forced_backends: bool = True, flashattention: bool = True) -> list[dict]:
    """Rows of benchmark_results.csv for the grid (run_study.py:482-648)."""
    import torch

    rows = []
    for causal in causal_flags:
        for dtype_name in dtypes:
            dtype = getattr(torch, dtype_name)
            for s in s_values:
                for d in d_values:
                    torch.manual_seed(1234)
                    q = torch.randn((b, h, s, d), device="cuda", dtype=dtype)
                    k = torch.randn((b, h, s, d), device="cuda", dtype=dtype)
                    v = torch.randn((b, h, s, d), device="cuda", dtype=dtype)
                    flops = attention_forward_flops(b=b, h=h, s=s, d=d, causal=causal)
                    stats = {}
                    for method, fn in build_methods(q, k, v, causal=causal, forced_backends=forced_backends,
                                                    flashattention=flashattention):
                        stats[method] = time_method(method, fn, warmup=warmup, iters=iters)
                    for method, (med, tail, status, detail) in stats.items():
                        rows.append({
                            "method": method, "baseline_name": BASELINE_NAME, "dtype": dtype_name,
                            "causal": causal, "B": b, "H": h, "S": s, "D": d, "flops_forward": flops,
                            "median_ms": med, "p95_ms": tail,
                            "throughput_tokens_per_s": throughput_tokens_per_s(b=b, h=h, s=s, median_ms=med),
                            "tflops_per_s": tflops_per_s(flops=flops, median_ms=med),
                            "approx_bw_gbps": approximate_bw_gbps(b=b, h=h, s=s, d=d, bytes_per_elem=2,
                                                                  median_ms=med),
                            "status": status, "status_detail": detail,
                        })
                    print(f"[study] causal={causal} dtype={dtype_name} S={s} D={d} "
                          + " ".join(f"{m}={r[0]:.3f}ms" for m, r in stats.items()), flush=True)
                    del q, k, v
    return rows


def run_tune(*, b: int, h: int, warmup: int, iters: int, regimes=TUNE_REGIMES,
             candidates=TUNE_CANDIDATES, d: int = 128) -> list[dict]:
    """Rows of tuning_results.csv: per regime the best and runner-up (TILE_M, TILE_N) of this
    package's kernels, fp16 non-causal fp32 accumulation (run_study.py:1230-1342).  Tiles this
    build does not have are skipped (they raise before launching)."""
    import torch

    from . import sdpa

    rows = []
    for name, s in regimes:
        torch.manual_seed(2026 + s)
        q = torch.randn((b, h, s, d), device="cuda", dtype=torch.float16)
        k = torch.randn((b, h, s, d), device="cuda", dtype=torch.float16)
        v = torch.randn((b, h, s, d), device="cuda", dtype=torch.float16)
        measured = []
        for tm, tn in candidates:
            env = {"TILEDATTN_TILE_M": str(tm), "TILEDATTN_TILE_N": str(tn), "TILEDATTN_ACCUM_MODE": "fp32"}
            old = {key: os.environ.get(key) for key in env}
            os.environ.update(env)
            try:
                med, _, status, detail = time_method("tiledattention", lambda: sdpa(q, k, v, causal=False),
                                                     warmup=warmup, iters=iters)
            finally:
                for key, val in old.items():
                    if val is None:
                        os.environ.pop(key, None)
                    else:
                        os.environ[key] = val
            print(f"[tune] {name} S={s} TM={tm} TN={tn} median={med:.3f}ms {status} {detail}", flush=True)
            if status == "ok":
                measured.append((med, tm, tn))
        measured.sort()
        best = measured[0]
        runner = measured[1] if len(measured) > 1 else measured[0]
        rows.append({
            "regime": name, "S": s, "D": d, "best_TM": best[1], "best_TN": best[2],
            "best_median_ms": best[0], "runner_TM": runner[1], "runner_TN": runner[2],
            "runner_median_ms": runner[0],
            "sensitivity_drop_percent": 100.0 * (runner[0] - best[0]) / best[0],
        })
        del q, k, v
    return rows


# ---------------------------------------------------------------- writers

def write_csv(path: Path, rows: list[dict], fields: tuple[str, ...]) -> None:
    if not rows:
        raise ValueError("rows must not be empty")
    with Path(path).open("w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(fields))
        w.writeheader()
        for r in rows:
            w.writerow({k: r[k] for k in fields})


def collect_repro_info() -> dict[str, str]:
    """Platform facts for table3_reproducibility.md (run_study.py:398-452, ROCm names)."""
    info = {"system": "Unknown", "driver": "Unknown", "rocm": "Unknown"}
    try:
        import torch

        info["torch"] = torch.__version__
        info["hip"] = str(torch.version.hip)
        if torch.cuda.is_available():
            prop = torch.cuda.get_device_properties(0)
            info["system"] = f"Host GPU: {prop.name} ({getattr(prop, 'gcnArchName', '?')})"
    except Exception as exc:  # pragma: no cover - reported, not fatal
        info["torch"] = f"Unavailable ({exc})"
    try:
        rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / ".info" / "version"
        info["rocm"] = rocm.read_text().strip()
    except Exception:
        pass
    try:
        out = subprocess.run(["hipcc", "--version"], capture_output=True, text=True, timeout=30).stdout
        info["hipcc"] = next((ln.strip() for ln in out.splitlines() if "HIP version" in ln), "Unknown")
    except Exception:
        info["hipcc"] = "Unavailable in PATH"
    from . import __version__

    info["tiledattention"] = __version__
    info["flashattention"] = "installed" if _flash_attn_func() is not None else \
        "Not installed (baseline used: torch SDPA)"
    info["host"] = f"{platform.machine()} {platform.system()} {platform.release()}"
    info["timing"] = "GPU events, median + p95 after warmup"
    return info


def write_table3(path: Path, info: dict[str, str]) -> None:
    lines = ["# Table 3: Reproducibility", "", "| Item | Value |", "| --- | --- |"]
    lines += [f"| {k} | {v} |" for k, v in info.items()]
    Path(path).write_text("\n".join(lines) + "\n")


def _fmt(x) -> str:
    return "nan" if isinstance(x, float) and math.isnan(x) else (f"{x:.3f}" if isinstance(x, float) else str(x))


def write_summary(path: Path, rows: list[dict], tune_rows: list[dict] | None = None) -> None:
    """Per-case table: this package against the baseline, speedup = baseline median / ours."""
    lines = ["# Study summary", "", f"Baseline: `{BASELINE_NAME}`.", "",
             "| dtype | causal | S | D | tiledattention ms | TFLOP/s | baseline ms | speedup | status |",
             "| --- | --- | --- | --- | --- | --- | --- | --- | --- |"]
    by_case: dict[tuple, dict[str, dict]] = {}
    for r in rows:
        by_case.setdefault((r["dtype"], r["causal"], r["S"], r["D"]), {})[r["method"]] = r
    for (dt, causal, s, d), m in by_case.items():
        ours, base = m.get("tiledattention"), m.get(BASELINE_NAME)
        if ours is None:
            continue
        sp = math.nan
        if base is not None and ours["median_ms"] == ours["median_ms"] and base["median_ms"] == base["median_ms"]:
            sp = base["median_ms"] / ours["median_ms"]
        lines.append(f"| {dt} | {causal} | {s} | {d} | {_fmt(ours['median_ms'])} | {_fmt(ours['tflops_per_s'])} "
                     f"| {_fmt(base['median_ms']) if base else 'n/a'} | {_fmt(sp)} | {ours['status']} |")
    if tune_rows:
        lines += ["", "## Tiling sensitivity", "",
                  "| regime | S | best (TM, TN) | best ms | runner-up | runner ms | drop % |",
                  "| --- | --- | --- | --- | --- | --- | --- |"]
        for t in tune_rows:
            lines.append(f"| {t['regime']} | {t['S']} | ({t['best_TM']}, {t['best_TN']}) | {_fmt(t['best_median_ms'])} "
                         f"| ({t['runner_TM']}, {t['runner_TN']}) | {_fmt(t['runner_median_ms'])} "
                         f"| {_fmt(t['sensitivity_drop_percent'])} |")
    Path(path).write_text("\n".join(lines) + "\n")


# ---------------------------------------------------------------- rocprofv3 summary

def _read_csv(path: Path) -> list[dict]:
    with Path(path).open(newline="") as f:
        return list(csv.DictReader(f))


def rocprof_metrics(prof_dir: Path, kernel_substring: str) -> dict[str, float | str | None]:
    """Primary-kernel metrics from a ``rocprofv3 -d DIR -o run`` tree: kernel time from
    ``*kernel_stats.csv`` and, where present, per-dispatch means of the counters in every
    ``*counter_collection.csv`` below it (summed over counter dimensions)."""
    prof_dir = Path(prof_dir)
    m: dict[str, float | str | None] = {"kernel": None, "kernel_ms": None}
    for stats in prof_dir.rglob("*kernel_stats.csv"):
        for r in _read_csv(stats):
            if kernel_substring in r["Name"]:
                m["kernel"] = r["Name"]
                m["kernel_ms"] = float(r["AverageNs"]) / 1e6
    sums: dict[str, dict[str, float]] = {}
    for cc in prof_dir.rglob("*counter_collection.csv"):
        for r in _read_csv(cc):
            if kernel_substring not in r["Kernel_Name"]:
                continue
            m["kernel"] = m["kernel"] or r["Kernel_Name"]
            sums.setdefault(r["Counter_Name"], {}).setdefault(r["Dispatch_Id"], 0.0)
            sums[r["Counter_Name"]][r["Dispatch_Id"]] += float(r["Counter_Value"])
    for name, per in sums.items():
        m[name] = sum(per.values()) / len(per)
    return m


def kernel_trace_table(prof_dir: Path, kernel_substring: str = "ta_fwd") -> list[dict]:
    """Per (kernel, workgroups) dispatch durations from every ``*kernel_trace.csv`` below a
    ``rocprofv3 --kernel-trace`` tree: calls, median, min and mean in microseconds.  One
    kernel symbol can run several workloads (grid sizes), which ``*kernel_stats.csv`` lumps
    together."""
    durs: dict[tuple[str, int], list[float]] = {}
    for trace in Path(prof_dir).rglob("*kernel_trace.csv"):
        for r in _read_csv(trace):
            name = r["Kernel_Name"]
            if kernel_substring not in name:
                continue
            wg = int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"]))
            durs.setdefault((name, wg), []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    return [{"kernel": k, "workgroups": wg, "calls": len(v), "median_us": statistics.median(v),
             "min_us": min(v), "mean_us": statistics.mean(v)} for (k, wg), v in sorted(durs.items())]


def write_kernel_trace_table(path: Path, rows: list[dict], config: dict[str, object]) -> None:
    lines = ["# rocprofv3 kernel trace: dispatch durations per kernel and grid", ""]
    lines += [f"- {k}: {v}" for k, v in config.items()]
    lines += ["", "| kernel | workgroups | calls | median us | min us | mean us |", "|---|---|---|---|---|---|"]
    lines += [f"| {r['kernel']} | {r['workgroups']} | {r['calls']} | {r['median_us']:.2f} | {r['min_us']:.2f} | "
              f"{r['mean_us']:.2f} |" for r in rows]
    Path(path).write_text("\n".join(lines) + "\n")


def _ratio(m, a, b, scale=100.0):
    x, y = m.get(a), m.get(b)
    return None if x is None or not y else scale * x / y


# MI355X: 8 XCDs (GRBM_GUI_ACTIVE is summed over them), 1024 SIMDs (SQ_VALU_MFMA_BUSY_CYCLES
# is summed over them), 32 SIMDs per shader engine (SQ_BUSY_CYCLES is summed over engines).
_XCDS, _SIMDS, _SIMDS_PER_SE = 8, 1024, 32


def mfma_busy_pct(m: dict) -> float | None:
    """MFMA-busy share of kernel cycles per SIMD: against GRBM_GUI_ACTIVE when measured, else
    against the shader engines' busy cycles."""
    busy = m.get("SQ_VALU_MFMA_BUSY_CYCLES")
    if busy is None:
        return None
    if m.get("GRBM_GUI_ACTIVE"):
        return 100.0 * busy / (m["GRBM_GUI_ACTIVE"] / _XCDS * _SIMDS)
    return _ratio(m, "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CYCLES", 100.0 / _SIMDS_PER_SE)


def diagnose(m: dict) -> list[str]:
    """Coarse bottleneck hints from the counters, in the spirit of run_ncu_profile.py:440-466."""
    lines = []
    mfma = mfma_busy_pct(m)
    wait = _ratio(m, "SQ_WAIT_ANY", "SQ_WAVE_CYCLES")
    lds_wait = _ratio(m, "SQ_WAIT_INST_LDS", "SQ_WAVE_CYCLES")
    if m.get("SQ_INSTS_MFMA") is not None and m["SQ_INSTS_MFMA"] < 1.0:
        lines.append("Near-zero MFMA activity on the primary kernel.")
    if mfma is not None and mfma < 30.0:
        lines.append("MFMA busy below 30 % of cycles: the matrix cores are underfed.")
    if wait is not None and wait > 30.0:
        lines.append("Waves wait in more than 30 % of their cycles (barriers, memory counters).")
    if lds_wait is not None and lds_wait > 10.0:
        lines.append("LDS waits above 10 % of wave cycles: LDS bandwidth or latency bound.")
    if m.get("SQ_LDS_BANK_CONFLICT"):
        lines.append("LDS bank conflicts present: check the LDS layout.")
    if not lines:
        lines.append("No single dominant bottleneck from coarse counters; see the kernel trace.")
    return lines


def write_rocprof_summary(path: Path, results: list[tuple[str, dict]], config: dict[str, object]) -> None:
    """Markdown summary shaped like the reference's Nsight one-pass summary."""
    lines = ["# rocprofv3 One-Pass Summary", "", "## Run Configuration", ""]
    lines += [f"- {k}: {v}" for k, v in config.items()]
    lines += ["", "## Key Metrics (primary kernel row)", "",
              "| Method | Primary Kernel | Kernel Time (ms) | MFMA Busy % | VALU Co-issue % of MFMA | "
              "Wait % | LDS Wait % | LDS Bank Conflicts | FETCH_SIZE KiB | WRITE_SIZE KiB |",
              "| --- | --- | --- | --- | --- | --- | --- | --- | --- | --- |"]

    def f(x):
        return "n/a" if x is None else (f"{x:.3f}" if isinstance(x, float) else str(x))

    for method, m in results:
        lines.append(
            f"| {method} | `{m.get('kernel')}` | {f(m.get('kernel_ms'))} | "
            f"{f(mfma_busy_pct(m))} | "
            f"{f(_ratio(m, 'SQ_VALU_MFMA_COEXEC_CYCLES', 'SQ_VALU_MFMA_BUSY_CYCLES'))} | "
            f"{f(_ratio(m, 'SQ_WAIT_ANY', 'SQ_WAVE_CYCLES'))} | {f(_ratio(m, 'SQ_WAIT_INST_LDS', 'SQ_WAVE_CYCLES'))} | "
            f"{f(m.get('SQ_LDS_BANK_CONFLICT'))} | {f(m.get('FETCH_SIZE'))} | {f(m.get('WRITE_SIZE'))} |")
    lines += ["", "## Counters (mean per dispatch, summed over counter dimensions)", "",
              "| Method | Counter | Mean |", "| --- | --- | --- |"]
    for method, m in results:
        for name in sorted(k for k in m if k not in ("kernel", "kernel_ms")):
            lines.append(f"| {method} | {name} | {f(m[name])} |")
    lines += ["", "## Quick Diagnosis", ""]
    for method, m in results:
        lines += [f"### {method}", "", f"- Primary kernel: `{m.get('kernel')}`",
                  f"- Kernel time (average over dispatches, ms): {f(m.get('kernel_ms'))}"]
        lines += [f"- {x}" for x in diagnose(m)]
        lines.append("")
    Path(path).write_text("\n".join(lines).rstrip() + "\n")


# ---------------------------------------------------------------- CLI

def _args(argv=None):
    ap = argparse.ArgumentParser(description="TiledAttention study on gfx950 (reference study schema).")
    ap.add_argument("--out", default="study_results", help="output directory")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--iters", type=int, default=15)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--heads", type=int, default=8)
    ap.add_argument("--seqs", type=int, nargs="+", default=[512, 1024, 2048, 4096, 8192])
    ap.add_argument("--dims", type=int, nargs="+", default=[64, 96, 128, 160])
    ap.add_argument("--dtypes", nargs="+", default=["float16", "bfloat16"])
    ap.add_argument("--no-causal", action="store_true")
    ap.add_argument("--disable-flashattention", action="store_true")
    ap.add_argument("--disable-forced-sdpa-backends", action="store_true")
    ap.add_argument("--no-tune", action="store_true")
    ap.add_argument("--rocprof-dir", default=None,
                    help="summarise an existing rocprofv3 output tree instead of benchmarking")
    ap.add_argument("--kernel", default="ta_fwd", help="primary-kernel name filter for --rocprof-dir")
    ap.add_argument("--trace-table", action="store_true",
                    help="with --rocprof-dir: also write kernel_trace.md (durations per kernel and grid)")
    return ap.parse_args(argv)


def main(argv=None) -> int:
    args = _args(argv)
    out = Path(args.out)
    out.mkdir(parents=True, exist_ok=True)
    if args.rocprof_dir:
        m = rocprof_metrics(Path(args.rocprof_dir), args.kernel)
        write_rocprof_summary(out / "rocprof_summary.md", [("tiledattention", m)],
                              {"rocprofv3 output": args.rocprof_dir, "kernel filter": args.kernel})
        print(f"[study] wrote {out / 'rocprof_summary.md'}")
        if args.trace_table:
            write_kernel_trace_table(out / "kernel_trace.md", kernel_trace_table(Path(args.rocprof_dir), args.kernel),
                                     {"rocprofv3 output": args.rocprof_dir, "kernel filter": args.kernel})
            print(f"[study] wrote {out / 'kernel_trace.md'}")
        return 0
    import torch

    if not torch.cuda.is_available():
        print("No GPU is available. Run this study on the host GPU.", file=sys.stderr)
        return 2
    causal_flags = [False] if args.no_causal else [False, True]
    print(f"[study] warmup={args.warmup} iters={args.iters} B={args.batch} H={args.heads} causal={causal_flags}",
          flush=True)
    rows = run_benchmark(b=args.batch, h=args.heads, s_values=args.seqs, d_values=args.dims, dtypes=args.dtypes,
                         causal_flags=causal_flags, warmup=args.warmup, iters=args.iters,
                         forced_backends=not args.disable_forced_sdpa_backends,
                         flashattention=not args.disable_flashattention)
    write_csv(out / "benchmark_results.csv", rows, BENCH_FIELDS)
    tune_rows = None
    if not args.no_tune:
        tune_rows = run_tune(b=args.batch, h=args.heads, warmup=args.warmup, iters=args.iters)
        write_csv(out / "tuning_results.csv", tune_rows, TUNE_FIELDS)
    write_table3(out / "table3_reproducibility.md", collect_repro_info())
    write_summary(out / "study_summary.md", rows, tune_rows)
    print("[study] completed", flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
