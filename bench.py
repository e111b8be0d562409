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
* ``sweep``: the C3 sequence sweep S in {512..8192}, kernel TFLOP/s and share of peak.

Usage: ``python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]``.
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


def _args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--seq", type=int, default=8192, help="sequence length of the headline workload")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--traffic-json", default=str(ROOT / "profiles" / "traffic.json"),
                    help="HBM bytes per launch measured by rocprofv3 (optional)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="also run a plain device copy of this many MiB (calibrates rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE against a known byte count)")
    return ap.parse_args()


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


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


def cpu_baseline(shape, dtype: str, seed: int, causal: bool, budget_s: float):
    """Time the eager restatement on host cores over whole (b, h) slices of the workload."""
    import torch

    from oracle import eager
    from oracle import oracle as O

    threads = min(os.cpu_count() or 1, 16)
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
        "cpu_model": platform.processor() or platform.machine(),
        "os_cpu_count": os.cpu_count(),
    }


def main() -> int:
    args = _args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported in this build "
              "(every GPU box here has one GPU).", file=sys.stderr)
        return 2

    import torch

    from oracle import oracle as O
    from tiledattention_amd import _lib, sdpa
    from tiledattention_amd.kernels import flash_fwd

    dev = torch.device("cuda:0")
    b, h, s, d = 1, 8, args.seq, 128
    dtype, causal, seed = "bfloat16", True, 1234
    _log(f"workload C3 B={b} H={h} S={s} D={d} {dtype} causal seed={seed}")
    q, k, v = (t.to(dev) for t in O.make_inputs((b, h, s, d), dtype, seed))
    flops = O.attention_forward_flops(b=b, h=h, s=s, d=d, causal=causal)
    nbytes = O.approximate_bytes(b=b, h=h, s=s, d=d, bytes_per_elem=2)

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

    # The kernel this configuration launches (the C ABI's choice, mirrored in _lib); the
    # committed HBM-traffic figure is used only if it was measured on that kernel.
    tm, tn = flash_fwd._default_tile_config_for_shape_gfx950(seq_len=s, head_dim=d, causal=causal)
    _, kernel = _lib.kernel_symbol(dtype=_lib.TA_BF16, head_dim=d, tile_m=tm, tile_n=tn,
                                   causal=causal, tail=(s % tm != 0 or s % tn != 0),
                                   accum=_lib.TA_ACC_FP32)
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
            qs, ks, vs = (t.to(dev) for t in O.make_inputs((1, 8, ss, 128), dtype, seed))
            f = O.attention_forward_flops(b=1, h=8, s=ss, d=128, causal=True)
            fn_s = lambda: sdpa(qs, ks, vs, causal=True)  # noqa: E731
            # The clocks drop under the light load of the smaller sizes and take tens of
            # milliseconds of sustained work to come back: 0.2 s of this size first, then the
            # median over five regions of ten back-to-back launches.
            t_end = time.perf_counter() + 0.2
            while time.perf_counter() < t_end:
                for _ in range(10):
                    fn_s()
                torch.cuda.synchronize()
            mean_s = statistics.median(time_kernel(fn_s, steps=10, warmup=0)[1] for _ in range(5))
            per_s = time_calls(fn_s, steps=50, warmup=0)
            sweep[str(ss)] = {
                "tflops": round(f / (mean_s * 1e-3) / 1e12, 2),
                "frac_peak": round(f / (mean_s * 1e-3) / 1e12 / PEAK_TFLOPS, 4),
                "mean_ms": round(mean_s, 5),
                "p95_ms": round(O.p95(per_s), 5),
                "hbm_gbps_alg": round(O.approximate_bytes(b=1, h=8, s=ss, d=128, bytes_per_elem=2)
                                      / (mean_s * 1e-3) / 1e9, 1),
            }
            _log(f"sweep S={ss}: {sweep[str(ss)]}")
            del qs, ks, vs

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
            "tile_m": tm, "tile_n": tn, "accum": "fp32", "kernel": kernel,
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
