"""Helpers shared by the GPU parity tests: seeded inputs, oracle comparison, env knobs.

Tolerances (max-abs against the explicit fp32 oracle, from the north star): 2e-3 for
fp16, 1e-2 for bf16.  Input-dtype accumulation (TILEDATTN_ACCUM_MODE=fp16) rounds O to the
input dtype after every key tile, as the reference does (flash_fwd.py:360-362); it is held
to 2.5x those bounds against the fp32 oracle and to the input dtype's own rounding against
the oracle's restatement of that rounding sequence (``flash_tiled(accum_lowp=True)``).
"""

from __future__ import annotations

import contextlib
import os
import sys

import numpy as np

from oracle import oracle as O

TOL = {"float16": 2e-3, "bfloat16": 1e-2}
LOWP_TOL = {"float16": 5e-3, "bfloat16": 2.5e-2}


def say(msg: str) -> None:
    """Name the case on stdout before any GPU work (flushed, so a crash still shows it)."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@contextlib.contextmanager
def knobs(**env):
    """Temporarily set TILEDATTN_* env knobs (values None = unset)."""
    old = {}
    for key, val in env.items():
        name = "TILEDATTN_" + key.upper()
        old[name] = os.environ.get(name)
        if val is None:
            os.environ.pop(name, None)
        else:
            os.environ[name] = str(val)
    try:
        yield
    finally:
        for name, val in old.items():
            if val is None:
                os.environ.pop(name, None)
            else:
                os.environ[name] = val


def inputs(shape, dtype, seed, **kw):
    q, k, v = O.make_inputs(shape, dtype, seed, **kw)
    return q, k, v


def run_gpu(q, k, v, *, causal, scale=None, **env):
    import torch

    from tiledattention import sdpa

    dev = torch.device("cuda:0")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    with knobs(**env):
        out = sdpa(qd, kd, vd, causal=causal, scale=scale)
    torch.cuda.synchronize()
    return out


def kernel_for(q, k, v, *, causal, **env) -> str:
    """The attention kernel the library launches for these inputs under the given knobs
    (``describe_call``, i.e. ``ta_describe_launch``); nothing is launched."""
    import torch

    from tiledattention.kernels import flash_fwd

    dev = torch.device("cuda:0")
    with knobs(**env):
        return flash_fwd.describe_call(q.to(dev), k.to(dev), v.to(dev), causal=causal).get("kernel", "")


def oracle_f32(q, k, v, *, causal, scale=None, rows=None):
    dc = O.dtype_code(str(q.dtype))
    qb, kb, vb = O.to_bits(q), O.to_bits(k), O.to_bits(v)
    return O.explicit_f32(qb, kb, vb, dc, causal=causal, scale=scale, rows=rows)


def as_f32(out, rows=None):
    """The output as fp32 numpy, optionally only the query rows `rows`.

    With `rows`, every element of the whole output is first checked for finiteness on its
    own device, so a NaN or inf outside the sampled rows still fails the test (the values
    of unsampled rows are not compared with the oracle, their finiteness is)."""
    import torch

    if rows is not None:
        bad = int((~torch.isfinite(out.detach())).sum())
        assert bad == 0, f"{bad} non-finite output elements (the whole output is checked)"
    o = out.detach().to("cpu", torch.float32)
    if rows is not None:
        o = o[:, :, torch.as_tensor(rows, dtype=torch.long), :]
    return o.contiguous().numpy()


def check_close(got: np.ndarray, ref: np.ndarray, dtype: str, tol: float | None = None, what: str = ""):
    """Assert max-abs error <= tol; returns the error."""
    t = TOL[dtype] if tol is None else tol
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = float(np.abs(got.astype(np.float64) - ref.astype(np.float64)).max()) if got.size else 0.0
    print(f"[check] {what} dtype={dtype} max_abs_err={err:.3e} tol={t:.1e}", flush=True)
    assert err <= t, f"{what}: max abs error {err:.3e} > {t:.1e}"
    return err


def sample_rows(s: int, n: int, seed: int = 7) -> np.ndarray:
    """First 64 rows, last 64 rows, and n random rows in between (sorted, unique)."""
    rng = np.random.default_rng(seed)
    head = np.arange(min(64, s))
    tail = np.arange(max(0, s - 64), s)
    mid = rng.choice(s, size=min(n, s), replace=False)
    return np.unique(np.concatenate([head, tail, mid])).astype(np.int64)
