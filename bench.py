"""Benchmark of the SDPA forward on one MI355X (the driver's bench contract).

Headline workload: C3 at S=8192 - B=1, H=8, S=8192, D=128,
bf16, causal, seed 1234, default knobs.  A "step" is one forward over that batch with the
inputs already resident in HBM.  Work per step is 4*B*H*S^2*D FLOPs halved for causal
(137.4 GFLOP), so ``value`` is TFLOP/s.

The JSON line also carries:

* ``roofline``: the attention kernel's achieved TFLOP/s (algorithmic FLOPs per launch /
  mean launch duration: two HIP events on the launch stream around the timed region's K
  back-to-back launches, divided by K) against the dense bf16 MFMA peak, 2516.6 TFLOP/s
  (256 CU x 4096 FLOP/clk x 2.4 GHz); ``traffic`` is the HBM bytes per launch measured with
  rocprofv3 counters (profiles/), or null when not measured in this run;
* ``cpu_baseline``: the reference's eager attention restated on the host CPU
  (oracle/eager.py, run_study.py:304-335) on a bounded sample of the same workload;
* ``sweep``: the C3 sequence sweep S in {512..8192} (bf16), as before;
* ``blocks``: every other BASELINE.json configuration, each timed the same way (TFLOP/s,
  share of peak, algorithmic HBM GB/s, mean and p95 per call, the kernel the library
  launches): C2, the C4 tile x accumulation sweep (fp16/bf16, D 64/128), C5 and its outlier
  variant C5b; ``grid``, the metric's curves: B1 H8, S in {512..8192}, fp16 and bf16, causal
  and not, D 64 and 128, each point beside the reference's own GB10 number
  (benchmark-gb10/results/benchmark_results.csv, line cited per point); ``ceiling``, what
  bounds the headline on the same box in the same run: hipBLASLt's bf16 GEMM (torch.matmul,
  8192^3) and the headline workload on inputs whose mantissas are cleared (same
  instructions and memory traffic, least multiplier activity); ``small``, grids of one to
  four heads at S 2048/4096 (bf16, D 64 and 128, causal and not), the default call policy
  beside whole 64-row blocks and the 128-row tile's own plan.

Inputs are generated on the CPU from a seeded ``torch.Generator`` (q, k, v drawn in that
order, as run_study.py:526-529 does) and copied to the GPU before any timing.

Usage: ``python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
[--no-sweep] [--no-blocks] [--only-block NAME]``.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

PEAK_TFLOPS = 2516.6  # dense fp16/bf16 MFMA, MI355X: 256 CU * 4096 FLOP/clk * 2.4 GHz
REFERENCE_GB10_C3_S8192 = 60.87  # benchmark-gb10/results/benchmark_results.csv:548, TFLOP/s
C4_TILES = ((64, 64), (64, 128), (128, 64), (128, 128))
GRID_S = (512, 1024, 2048, 4096, 8192)

# The reference's TFLOP/s on GB10 for its B1 H8 grid (method "tiledattention"), keyed by
# (dtype, causal, S, D): (line of benchmark-gb10/results/benchmark_results.csv, TFLOP/s).
REFERENCE_GB10_GRID = {
    ("float16", False, 512, 64): (2, 15.197), ("float16", False, 512, 128): (16, 24.123),
    ("float16", False, 1024, 64): (30, 34.222), ("float16", False, 1024, 128): (44, 46.929),
    ("float16", False, 2048, 64): (58, 48.115), ("float16", False, 2048, 128): (72, 60.241),
    ("float16", False, 4096, 64): (86, 58.803), ("float16", False, 4096, 128): (100, 70.232),
    ("float16", False, 8192, 64): (114, 61.928), ("float16", False, 8192, 128): (128, 71.119),
    ("bfloat16", False, 512, 64): (142, 15.636), ("bfloat16", False, 512, 128): (156, 23.334),
    ("bfloat16", False, 1024, 64): (170, 35.209), ("bfloat16", False, 1024, 128): (184, 44.311),
    ("bfloat16", False, 2048, 64): (198, 48.586), ("bfloat16", False, 2048, 128): (212, 57.796),
    ("bfloat16", False, 4096, 64): (226, 59.020), ("bfloat16", False, 4096, 128): (240, 67.056),
    ("bfloat16", False, 8192, 64): (254, 61.970), ("bfloat16", False, 8192, 128): (268, 68.317),
    ("float16", True, 512, 64): (282, 8.904), ("float16", True, 512, 128): (296, 15.240),
    ("float16", True, 1024, 64): (310, 21.641), ("float16", True, 1024, 128): (324, 32.420),
    ("float16", True, 2048, 64): (338, 37.218), ("float16", True, 2048, 128): (352, 50.012),
    ("float16", True, 4096, 64): (366, 48.166), ("float16", True, 4096, 128): (380, 61.523),
    ("float16", True, 8192, 64): (394, 53.977), ("float16", True, 8192, 128): (408, 63.994),
    ("bfloat16", True, 512, 64): (422, 8.894), ("bfloat16", True, 512, 128): (436, 15.158),
    ("bfloat16", True, 1024, 64): (450, 21.097), ("bfloat16", True, 1024, 128): (464, 31.186),
    ("bfloat16", True, 2048, 64): (478, 36.040), ("bfloat16", True, 2048, 128): (492, 47.805),
    ("bfloat16", True, 4096, 64): (506, 47.052), ("bfloat16", True, 4096, 128): (520, 58.014),
    ("bfloat16", True, 8192, 64): (534, 52.394), ("bfloat16", True, 8192, 128): (548, 60.875),
}


def _args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--seq", type=int, default=8192, help="sequence length of the headline workload")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-blocks", action="store_true", help="skip the other BASELINE configurations")
    ap.add_argument("--only-block", default="", help="run only blocks whose name starts with this")
    ap.add_argument("--traffic-json", default=str(ROOT / "profiles" / "traffic.json"),
                    help="HBM bytes per launch measured by rocprofv3 (optional)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="also run a plain device copy of this many MiB (calibrates rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE against a known byte count)")
    return ap.parse_args()


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------- workload definitions

def make_inputs(shape, dtype: str, seed: int, *, scale_inputs: float = 1.0, outlier_frac: float = 0.0,
                outlier_gain: float = 20.0, outlier_seed: int | None = None):
    """Seeded q, k, v (CPU tensors of ``dtype``): ``randn`` in fp32 from
    ``torch.Generator('cpu').manual_seed(seed)`` in the order q, k, v (run_study.py:526-529),
    times ``scale_inputs``; ``outlier_frac`` > 0 multiplies that fraction of k's entries,
    chosen uniformly with ``outlier_seed``, by ``outlier_gain`` (BASELINE config C5b)."""
    import torch

    tdt = {"float16": torch.float16, "bfloat16": torch.bfloat16}[dtype]
    g = torch.Generator(device="cpu").manual_seed(int(seed))
    q = torch.randn(shape, generator=g, dtype=torch.float32) * scale_inputs
    k = torch.randn(shape, generator=g, dtype=torch.float32) * scale_inputs
    v = torch.randn(shape, generator=g, dtype=torch.float32) * scale_inputs
    if outlier_frac > 0.0:
        g2 = torch.Generator(device="cpu").manual_seed(int(outlier_seed if outlier_seed is not None else seed + 1))
        idx = torch.randperm(k.numel(), generator=g2)[: int(round(k.numel() * outlier_frac))]
        flat = k.reshape(-1)
        flat[idx] = flat[idx] * outlier_gain
    return q.to(tdt), k.to(tdt), v.to(tdt)


def flops_of(b: int, h: int, s: int, d: int, causal: bool) -> float:
    """Work of one forward as BASELINE.json counts it: 4*B*H*S^2*D, halved when causal."""
    f = 4.0 * b * h * s * s * d
    return f / 2.0 if causal else f


def alg_bytes(b: int, h: int, s: int, d: int) -> float:
    """Algorithmic HBM bytes: q, k, v read and o written once, 2 bytes an element
    (run_study.py:146)."""
    return 4.0 * b * h * s * d * 2


def p95(values) -> float:
    """95th percentile as run_study.py:30-45 takes it (quantiles n=20, index 18)."""
    vals = list(values)
    return vals[0] if len(vals) == 1 else statistics.quantiles(vals, n=20)[18]


# ---------------------------------------------------------------- timing

def time_kernel(fn, *, steps: int, warmup: int):
    """Warm up, then time ``steps`` back-to-back calls: wall clock around the region
    (synchronized on both sides) and two HIP events on the launch stream around it.  Returns
    (wall ms per call, event ms per launch).  No event sits between the launches: an event
    record per call adds ~7 us of queue work per step on the MI355X and stretches the
    events' own reading of the kernel by ~2 us."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    return wall_ms / steps, e0.elapsed_time(e1) / steps


def time_calls(fn, *, steps: int, warmup: int):
    """Per-call durations (HIP events around every call on the launch stream), for a
    distribution; each event record adds its own queue work, so these read slightly long."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in ev:
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in ev]


def measure(fn, *, flops: float, nbytes: float, hot_s: float = 0.2, regions: int = 5, per_region: int = 10,
            calls: int = 50) -> dict:
    """Kernel time of ``fn``: ``hot_s`` seconds of the same work first (the clocks drop under
    light load and take tens of milliseconds of sustained work to come back), then the
    median over ``regions`` regions of ``per_region`` back-to-back launches; p95 over
    ``calls`` individually timed calls."""
    import torch

    t_end = time.perf_counter() + hot_s
    while time.perf_counter() < t_end:
        for _ in range(per_region):
            fn()
        torch.cuda.synchronize()
    mean_ms = statistics.median(time_kernel(fn, steps=per_region, warmup=0)[1] for _ in range(regions))
    per = time_calls(fn, steps=calls, warmup=0)
    tf = flops / (mean_ms * 1e-3) / 1e12
    return {
        "tflops": round(tf, 2),
        "frac_peak": round(tf / PEAK_TFLOPS, 4),
        "mean_ms": round(mean_ms, 5),
        "p95_ms": round(p95(per), 5),
        "hbm_gbps_alg": round(nbytes / (mean_ms * 1e-3) / 1e9, 1),
    }


class _Env:
    """Set TILEDATTN_* knobs for a block, restoring the previous values after it."""

    def __init__(self, **env):
        self.env = {"TILEDATTN_" + k.upper(): v for k, v in env.items()}
        self.old = {}

    def __enter__(self):
        for k, v in self.env.items():
            self.old[k] = os.environ.get(k)
            os.environ[k] = str(v)

    def __exit__(self, *exc):
        for k, v in self.old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def _describe(q, k, v, causal: bool) -> dict:
    """The launch the library makes for this call under the current knobs
    (``ta_describe_launch``); nothing is launched."""
    from tiledattention.kernels import flash_fwd

    return flash_fwd.describe_call(q, k, v, causal=causal)


def _kernel_of(q, k, v, causal: bool) -> str:
    """The attention kernel the library launches for this call."""
    return _describe(q, k, v, causal).get("kernel", "")


def clear_mantissa(t, keep_bits: int = 0):
    """``t`` (fp16/bf16) with all but the top ``keep_bits`` mantissa bits cleared: the same
    exponents and signs, so the same softmax ranges, with less multiplier activity."""
    import torch

    man = 7 if t.dtype == torch.bfloat16 else 10
    mask = (0xFFFF << (man - keep_bits)) & 0xFFFF
    bits = t.view(torch.int16).to(torch.int32) & mask
    return bits.to(torch.int16).view(t.dtype)


def run_blocks(dev, only: str = "") -> dict:
    """Every BASELINE.json configuration beside the headline, timed like the sweep."""
    import torch

    from tiledattention import sdpa

    blocks: dict = {}

    def want(name):
        return name.startswith(only) if only else True

    def one(name, shape, dtype, causal, seed, env=None, quiet=False, **input_kw):
        b, h, s, d = shape
        q, k, v = (t.to(dev) for t in make_inputs(shape, dtype, seed, **input_kw))
        with _Env(**(env or {})):
            fn = lambda: sdpa(q, k, v, causal=causal)  # noqa: E731
            rec = measure(fn, flops=flops_of(b, h, s, d, causal), nbytes=alg_bytes(b, h, s, d))
            rec["kernel"] = _kernel_of(q, k, v, causal)
        rec.update({"B": b, "H": h, "S": s, "D": d, "dtype": dtype, "causal": causal, "seed": seed})
        if env:
            rec["knobs"] = {("TILEDATTN_" + k.upper()): v for k, v in env.items()}
        if not quiet:
            _log(f"block {name}: {rec['tflops']} TFLOP/s ({rec['frac_peak']:.1%}), "
                 f"{rec['hbm_gbps_alg']} GB/s alg, p95 {rec['p95_ms']} ms, {rec['kernel']}")
        del q, k, v
        torch.cuda.empty_cache()
        return rec

    if want("C2"):
        # C2: B1 H8 S1024 D64 fp16 non-causal, tile 64x64, fp32 accumulation (aligned fast path)
        blocks["C2"] = one("C2", (1, 8, 1024, 64), "float16", False, 2026,
                           env={"tile_m": 64, "tile_n": 64, "accum_mode": "fp32"})
    if want("grid"):
        # The metric's curves (TFLOP/s vs S for fp16/bf16, D 64/128, causal and not) at the
        # reference's B1 H8 grid, seed 1234, default knobs, each beside the reference's point.
        grid = {}
        for dtype in ("float16", "bfloat16"):
            for causal in (False, True):
                for d in (64, 128):
                    curve = {}
                    for s_ in GRID_S:
                        rec = one("grid", (1, 8, s_, d), dtype, causal, 1234, quiet=True)
                        line_no, ref = REFERENCE_GB10_GRID[(dtype, causal, s_, d)]
                        rec["reference_gb10_tflops"] = ref
                        rec["reference_csv_line"] = line_no
                        rec["vs_reference"] = round(rec["tflops"] / ref, 2)
                        curve[str(s_)] = rec
                    key = f"{'fp16' if dtype == 'float16' else 'bf16'}_{'causal' if causal else 'noncausal'}_d{d}"
                    grid[key] = curve
                    _log(f"block grid {key}: " + ", ".join(
                        f"S={s_} {curve[str(s_)]['tflops']} ({curve[str(s_)]['frac_peak']:.1%}; ref "
                        f"{curve[str(s_)]['reference_gb10_tflops']})" for s_ in GRID_S))
        blocks["grid"] = grid
    if want("C4"):
        # C4: B4 H16 S4096 non-causal, inputs N(0,1)*0.5 seed 2026; every tile, both
        # accumulation modes; plus the default configuration (no knobs).
        c4 = {}
        for dtype in ("float16", "bfloat16"):
            for d in (64, 128):
                shape = (4, 16, 4096, d)
                q, k, v = (t.to(dev) for t in make_inputs(shape, dtype, 2026, scale_inputs=0.5))
                for tiles in (None,) + C4_TILES:
                    for acc in (("fp32",) if tiles is None else ("fp32", "fp16")):
                        key = f"{'fp16' if dtype == 'float16' else 'bf16'}_d{d}_" + (
                            "default" if tiles is None else f"{tiles[0]}x{tiles[1]}_{acc}")
                        env = {} if tiles is None else {"tile_m": tiles[0], "tile_n": tiles[1],
                                                         "accum_mode": acc}
                        with _Env(**env):
                            fn = lambda: sdpa(q, k, v, causal=False)  # noqa: E731
                            rec = measure(fn, flops=flops_of(*shape, False), nbytes=alg_bytes(*shape),
                                          hot_s=0.1, regions=3, per_region=10, calls=20)
                            rec["kernel"] = _kernel_of(q, k, v, False)
                        rec.update({"knobs": {("TILEDATTN_" + k_.upper()): v_ for k_, v_ in env.items()}})
                        c4[key] = rec
                        _log(f"block C4 {key}: {rec['tflops']} TFLOP/s ({rec['frac_peak']:.1%}) {rec['kernel']}")
                del q, k, v
                torch.cuda.empty_cache()
        for key, rec in c4.items():
            if not key.endswith("default"):
                rec["vs_default"] = round(rec["tflops"] / c4[key.rsplit("_", 2)[0] + "_default"]["tflops"], 3)
        blocks["C4"] = c4
    if want("C5"):
        blocks["C5"] = one("C5", (1, 8, 16384, 128), "float16", True, 1234)
        blocks["C5b"] = one("C5b", (1, 8, 16384, 128), "float16", True, 1234,
                            outlier_frac=0.01, outlier_gain=20.0, outlier_seed=1235)
    if want("ceiling"):
        blocks["ceiling"] = run_ceiling(dev)
    if want("small"):
        blocks["small"] = run_small_grids(dev)
    return blocks


# Small B*H grids (64-row blocks fill at most half the CUs): the default call policy beside
# the two plans it chooses between, bf16, seed 1234.
SMALL_GRIDS = ((1, 2048), (1, 4096), (2, 4096), (4, 2048))
SMALL_ALTERNATIVES = (
    ("whole64", {"tile_m": 64, "tile_n": 64, "split": "off"}),
    ("plan128", {"tile_m": 128, "tile_n": 64}),
)


def run_small_grids(dev) -> dict:
    """Default knobs against whole 64-row blocks and against the 128-row tile's own plan
    (its split or paired split), on grids of one to four heads: the range where the
    64-row kernel's key-range split is planned (``ta_split_plan_model_rows``)."""
    import torch

    from tiledattention import sdpa

    out: dict = {}
    for d in (64, 128):
        for causal in (False, True):
            for bh, s_ in SMALL_GRIDS:
                shape = (1, bh, s_, d)
                q, k, v = (t.to(dev) for t in make_inputs(shape, "bfloat16", 1234))
                row: dict = {}
                for label, env in (("default", {}),) + SMALL_ALTERNATIVES:
                    with _Env(**env):
                        fn = lambda: sdpa(q, k, v, causal=causal)  # noqa: E731
                        rec = measure(fn, flops=flops_of(*shape, causal), nbytes=alg_bytes(*shape),
                                      hot_s=0.1, regions=3, per_region=10, calls=20)
                        desc = _describe(q, k, v, causal)
                    row[label] = {"us": round(rec["mean_ms"] * 1e3, 2), "tflops": rec["tflops"],
                                  "kernel": desc.get("kernel", ""), "chunk_steps": desc.get("chunk_steps", 0)}
                for label, _ in SMALL_ALTERNATIVES:
                    row[label]["vs_default"] = round(row["default"]["us"] / row[label]["us"], 3)
                key = f"d{d}_{'causal' if causal else 'noncausal'}_bh{bh}_s{s_}"
                out[key] = row
                _log(f"block small {key}: default {row['default']['us']} us "
                     f"({row['default']['kernel']}/c{row['default']['chunk_steps']}), " + ", ".join(
                         f"{lb} {row[lb]['us']} us" for lb, _ in SMALL_ALTERNATIVES))
                del q, k, v
                torch.cuda.empty_cache()
    return out



def run_ceiling(dev) -> dict:
    """The headline kernel beside what bounds it, on the same box in the same run.

    * hipBLASLt's bf16 GEMM through torch.matmul, M = N = K = 8192 (and 16384): dense MFMA
      work with no softmax, the library's best rate on this part at this moment;
    * the headline workload (C3 S=8192 bf16 causal) on its own inputs, and on the same
      inputs with every mantissa bit cleared (and with 3 of bf16's 7 kept): the same
      kernel, instructions and memory traffic, only the operands' bit activity differs, so
      a rate that rises as bits are cleared is set by power (the clock the part holds),
      not by the schedule."""
    import torch

    from tiledattention import sdpa

    out: dict = {}
    for n in (8192, 16384):
        g = torch.Generator(device="cpu").manual_seed(7)
        a = torch.randn((n, n), generator=g, dtype=torch.float32).to(torch.bfloat16).to(dev)
        b_ = torch.randn((n, n), generator=g, dtype=torch.float32).to(torch.bfloat16).to(dev)
        c = torch.empty((n, n), dtype=torch.bfloat16, device=dev)
        fn = lambda: torch.matmul(a, b_, out=c)  # noqa: E731
        rec = measure(fn, flops=2.0 * n ** 3, nbytes=3.0 * n * n * 2, hot_s=0.5, regions=5,
                      per_region=5 if n == 8192 else 2, calls=10)
        out[f"gemm_bf16_{n}"] = rec
        _log(f"ceiling gemm bf16 {n}^3: {rec['tflops']} TFLOP/s ({rec['frac_peak']:.1%})")
        del a, b_, c
        torch.cuda.empty_cache()
    shape, causal = (1, 8, 8192, 128), True
    q, k, v = (t.to(dev) for t in make_inputs(shape, "bfloat16", 1234))
    flops = flops_of(*shape, causal)
    for label, keep in (("attention_c3_s8192", None), ("attention_c3_s8192_mantissa3", 3),
                        ("attention_c3_s8192_mantissa0", 0)):
        qi, ki, vi = (q, k, v) if keep is None else (clear_mantissa(t, keep) for t in (q, k, v))
        fn = lambda: sdpa(qi, ki, vi, causal=causal)  # noqa: E731
        rec = measure(fn, flops=flops, nbytes=alg_bytes(*shape), hot_s=0.5)
        rec["kernel"] = _kernel_of(qi, ki, vi, causal)
        out[label] = rec
        _log(f"ceiling {label}: {rec['tflops']} TFLOP/s ({rec['frac_peak']:.1%}) {rec['kernel']}")
    out["attention_vs_gemm_8192"] = round(out["attention_c3_s8192"]["tflops"] / out["gemm_bf16_8192"]["tflops"], 4)
    out["attention_vs_gemm_16384"] = round(out["attention_c3_s8192"]["tflops"] / out["gemm_bf16_16384"]["tflops"], 4)
    return out


def _cpu_model() -> str:
    """The host CPU's model string (``model name`` in /proc/cpuinfo)."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(shape, dtype: str, seed: int, causal: bool, budget_s: float):
    """Time the eager restatement on host cores over whole (b, h) slices of the workload,
    with every core this process may run on."""
    import torch

    from oracle import eager
    from oracle import oracle as O

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    q, k, v = O.make_inputs(shape, dtype, seed)
    b_, h_, s, d = shape
    pairs = [(b, h) for b in range(b_) for h in range(h_)]
    eager.eager_attention_per_head(q, k, v, causal=causal, heads=pairs[:1])  # warmup
    times = []
    start = time.perf_counter()
    i = 0
    while True:
        t0 = time.perf_counter()
        eager.eager_attention_per_head(q, k, v, causal=causal, heads=[pairs[i % len(pairs)]])
        times.append(time.perf_counter() - t0)
        i += 1
        if i >= 3 and time.perf_counter() - start > budget_s:
            break
        if i >= 200:
            break
    per_head = statistics.median(times)
    flops_head = O.attention_forward_flops(b=1, h=1, s=s, d=d, causal=causal)
    return {
        "value": flops_head / per_head / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"eager attention (run_study.py:304-335 restated, torch CPU {dtype}) on "
                   f"{len(times)} single-head slices of the workload, S={s} D={d}, median "
                   f"{per_head * 1e3:.1f} ms/head; same FLOP count as the GPU line"),
        "ms_per_head_median": per_head * 1e3,
        "ms_per_head_p95": O.p95([t * 1e3 for t in times]),
        "cpu_model": _cpu_model(),
        "os_cpu_count": os.cpu_count(),
    }


def main() -> int:
    args = _args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported in this build "
              "(every GPU box here has one GPU).", file=sys.stderr)
        return 2

    import torch

    from tiledattention import sdpa
    from tiledattention.kernels import flash_fwd

    dev = torch.device("cuda:0")
    b, h, s, d = 1, 8, args.seq, 128
    dtype, causal, seed = "bfloat16", True, 1234
    _log(f"workload C3 B={b} H={h} S={s} D={d} {dtype} causal seed={seed}")
    q, k, v = (t.to(dev) for t in make_inputs((b, h, s, d), dtype, seed))
    flops = flops_of(b, h, s, d, causal)
    nbytes = alg_bytes(b, h, s, d)

    def step():
        return sdpa(q, k, v, causal=causal)

    # Bring clocks up before any timing: ~0.5 s of the workload itself.
    t_end = time.perf_counter() + 0.5
    while time.perf_counter() < t_end:
        step()
        torch.cuda.synchronize()

    ms_step, kern_ms = time_kernel(step, steps=args.steps, warmup=args.warmup)
    value = flops / (ms_step * 1e-3) / 1e12
    achieved = flops / (kern_ms * 1e-3) / 1e12
    _log(f"ms/step {ms_step:.4f}  kernel mean {kern_ms:.4f} ms  "
         f"{value:.1f} TFLOP/s  kernel {achieved:.1f} TFLOP/s ({achieved / PEAK_TFLOPS:.1%} of peak)")

    # The kernel this configuration launches, as the library reports it; the committed
    # HBM-traffic figure is used only if it was measured on that kernel.
    desc = flash_fwd.describe_call(q, k, v, causal=causal)
    kernel = desc["kernel"]
    _log(f"headline kernel {kernel}: grid {desc['grid']} x {desc['block']}, layout {desc['layout']}")
    traffic = None
    tp = Path(args.traffic_json)
    if tp.exists():
        try:
            rec = json.loads(tp.read_text()).get(f"c3_s{s}")
            if rec and rec.get("kernel") == kernel:
                traffic = rec["hbm_bytes_per_launch"]
        except (ValueError, KeyError, TypeError):
            traffic = None

    sweep = {}
    if not args.no_sweep:
        for ss in (512, 1024, 2048, 4096, 8192):
            qs, ks, vs = (t.to(dev) for t in make_inputs((1, 8, ss, 128), dtype, seed))
            fn_s = lambda: sdpa(qs, ks, vs, causal=True)  # noqa: E731
            sweep[str(ss)] = measure(fn_s, flops=flops_of(1, 8, ss, 128, True), nbytes=alg_bytes(1, 8, ss, 128))
            sweep[str(ss)]["kernel"] = _kernel_of(qs, ks, vs, True)
            _log(f"sweep S={ss}: {sweep[str(ss)]}")
            del qs, ks, vs

    blocks = {} if args.no_blocks else run_blocks(dev, args.only_block)

    line = {
        "metric": "SDPA fwd TFLOP/s vs seq len (fp16/bf16, D=64/128) + % of MI355X MFMA peak",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / REFERENCE_GB10_C3_S8192, 3) if s == 8192 else None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v, CPU generator)",
        "config": {
            "workload": f"C3: sdpa fwd B={b} H={h} S={s} D={d} bf16 causal, seed {seed}",
            "B": b, "H": h, "S": s, "D": d, "causal": causal,
            "accum": "fp32", "kernel": kernel, "launch": desc,
            "flops_per_step": flops,
            "reference_value_gb10": REFERENCE_GB10_C3_S8192 if s == 8192 else None,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_TFLOPS, 4),
            "traffic": traffic,
            "kernel_mean_ms": round(kern_ms, 5),
            "alg_bytes": nbytes,
        },
        "sweep": sweep,
        "blocks": blocks,
    }

    if args.copy_probe_mib > 0:
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        line["copy_probe_bytes"] = n * 4
        del src, dst

    if not args.no_cpu_baseline:
        _log("cpu baseline (eager restatement on host cores)")
        line["cpu_baseline"] = cpu_baseline((b, h, s, d), dtype, seed, causal, args.cpu_seconds)
        _log(f"cpu baseline {line['cpu_baseline']['value']:.4f} TFLOP/s on {line['cpu_baseline']['cores']} threads")
    else:
        line["cpu_baseline"] = None

    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
