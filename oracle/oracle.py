"""CPU oracle for the SDPA forward path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker or the timed CPU
baseline; the operator in ``tiledattention`` never imports it and has no CPU fallback.

Contents:

* ``explicit_f32`` / ``explicit_f64`` - explicit softmax(QK^T*scale + mask)V, every step in
  fp32 (fp64), from the upcast fp16/bf16 inputs: the correctness oracle named by the
  north star.  C implementation in ``attention_oracle.c``.
* ``flash_tiled`` - restatement of the reference kernel's tiled online-softmax algorithm
  (src/tiledattention/kernels/flash_fwd.py:374-446, and :301-372 for accumulation in the
  input dtype), rounding to the input dtype exactly where the reference casts.
* ``make_inputs`` - seeded inputs as the benchmark harness draws them
  (benchmark-gb10/run_study.py:526-529: q, k, v from ``randn`` in that order), but on a CPU
  generator so that every device sees the same bits.
* ``attention_forward_flops`` / ``approximate_bytes`` / ``p95`` - the harness's work and
  statistics formulas (run_study.py:30-45, 95-148).

Parity pins for each function are listed in ``tests/test_oracle.py``.
"""

from __future__ import annotations

import ctypes
import math
import statistics
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

FP16 = 0
BF16 = 1

_lib = None


def build() -> Path:
    """Compile ``attention_oracle.c`` with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    u16p = ctypes.POINTER(ctypes.c_uint16)
    f32p = ctypes.POINTER(ctypes.c_float)
    f64p = ctypes.POINTER(ctypes.c_double)
    i64p = ctypes.POINTER(ctypes.c_int64)
    i64 = ctypes.c_int64
    cint = ctypes.c_int
    lib.ora_explicit_f32.argtypes = [u16p, u16p, u16p, cint, i64, i64, i64, cint, ctypes.c_float,
                                     i64p, i64, f32p]
    lib.ora_explicit_f32.restype = None
    lib.ora_explicit_f64.argtypes = [u16p, u16p, u16p, cint, i64, i64, i64, cint, ctypes.c_double,
                                     i64p, i64, f64p]
    lib.ora_explicit_f64.restype = None
    lib.ora_flash_tiled.argtypes = [u16p, u16p, u16p, cint, i64, i64, i64, cint, ctypes.c_float,
                                    i64, i64, cint, cint, cint, u16p]
    lib.ora_flash_tiled.restype = None
    lib.ora_round.argtypes = [f32p, u16p, i64, cint]
    lib.ora_round.restype = None
    lib.ora_upcast.argtypes = [u16p, f32p, i64, cint]
    lib.ora_upcast.restype = None
    _lib = lib
    return lib


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def dtype_code(name: str) -> int:
    """'float16'/'fp16' -> 0, 'bfloat16'/'bf16' -> 1."""
    n = str(name).replace("torch.", "")
    if n in ("float16", "fp16", "half"):
        return FP16
    if n in ("bfloat16", "bf16"):
        return BF16
    raise ValueError(f"unsupported dtype {name!r}")


def _bits(x: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(x)
    if a.dtype != np.uint16:
        raise TypeError("expected uint16 bit patterns")
    return a


def round_to(x: np.ndarray, dtype: int) -> np.ndarray:
    """fp32 array -> fp16/bf16 bit patterns, round to nearest even."""
    lib = _load()
    src = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(src.shape, dtype=np.uint16)
    lib.ora_round(_ptr(src, ctypes.c_float), _ptr(out, ctypes.c_uint16), src.size, dtype)
    return out


def upcast(bits: np.ndarray, dtype: int) -> np.ndarray:
    """fp16/bf16 bit patterns -> exact fp32 values."""
    lib = _load()
    src = _bits(bits)
    out = np.empty(src.shape, dtype=np.float32)
    lib.ora_upcast(_ptr(src, ctypes.c_uint16), _ptr(out, ctypes.c_float), src.size, dtype)
    return out


def _shape4(q: np.ndarray):
    if q.ndim != 4:
        raise ValueError("expected [B, H, S, D]")
    b, h, s, d = q.shape
    return b, h, s, d


def _rows_arg(rows):
    if rows is None:
        return None, 0
    r = np.ascontiguousarray(np.asarray(rows, dtype=np.int64))
    return r, r.size


def explicit_f32(q, k, v, dtype: int, *, causal: bool, scale: float | None = None, rows=None):
    """Explicit fp32 attention; returns fp32 [B,H,S,D] (or [B,H,len(rows),D])."""
    lib = _load()
    q, k, v = _bits(q), _bits(k), _bits(v)
    b, h, s, d = _shape4(q)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    r, nr = _rows_arg(rows)
    n_out = nr if r is not None else s
    out = np.empty((b, h, n_out, d), dtype=np.float32)
    lib.ora_explicit_f32(_ptr(q, ctypes.c_uint16), _ptr(k, ctypes.c_uint16), _ptr(v, ctypes.c_uint16),
                         dtype, b * h, s, d, int(causal), float(scale),
                         _ptr(r, ctypes.c_int64) if r is not None else None, nr,
                         _ptr(out, ctypes.c_float))
    return out


def explicit_f64(q, k, v, dtype: int, *, causal: bool, scale: float | None = None, rows=None):
    """Explicit fp64 attention (cross-check of ``explicit_f32``)."""
    lib = _load()
    q, k, v = _bits(q), _bits(k), _bits(v)
    b, h, s, d = _shape4(q)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    r, nr = _rows_arg(rows)
    n_out = nr if r is not None else s
    out = np.empty((b, h, n_out, d), dtype=np.float64)
    lib.ora_explicit_f64(_ptr(q, ctypes.c_uint16), _ptr(k, ctypes.c_uint16), _ptr(v, ctypes.c_uint16),
                         dtype, b * h, s, d, int(causal), float(scale),
                         _ptr(r, ctypes.c_int64) if r is not None else None, nr,
                         _ptr(out, ctypes.c_double))
    return out


def flash_tiled(q, k, v, dtype: int, *, causal: bool, scale: float | None = None,
                tile_m: int = 64, tile_n: int = 64, accum_lowp: bool = False,
                score_lowp: bool = False, l_rounded: bool = False) -> np.ndarray:
    """The reference kernel's tiled algorithm; returns fp16/bf16 bit patterns [B,H,S,D]."""
    lib = _load()
    q, k, v = _bits(q), _bits(k), _bits(v)
    b, h, s, d = _shape4(q)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    out = np.zeros((b, h, s, d), dtype=np.uint16)
    lib.ora_flash_tiled(_ptr(q, ctypes.c_uint16), _ptr(k, ctypes.c_uint16), _ptr(v, ctypes.c_uint16),
                        dtype, b * h, s, d, int(causal), float(scale), int(tile_m), int(tile_n),
                        int(accum_lowp), int(score_lowp), int(l_rounded), _ptr(out, ctypes.c_uint16))
    return out


# --------------------------------------------------------------------------- inputs

def make_inputs(shape, dtype: str, seed: int, *, scale_inputs: float = 1.0,
                outlier_frac: float = 0.0, outlier_gain: float = 20.0, outlier_seed: int | None = None):
    """Seeded q, k, v as torch CPU tensors of ``dtype``.

    q, k, v are drawn in that order with ``randn`` in fp32 from ``torch.Generator('cpu')``
    seeded with ``seed`` (order as in run_study.py:527-529), multiplied by
    ``scale_inputs`` and cast.  ``outlier_frac`` > 0 multiplies that fraction of k's
    entries, picked uniformly with ``outlier_seed``, by ``outlier_gain`` before the cast
    (the long-sequence outlier variant).
    """
    import torch

    tdt = {"float16": torch.float16, "fp16": torch.float16,
           "bfloat16": torch.bfloat16, "bf16": torch.bfloat16}[str(dtype).replace("torch.", "")]
    g = torch.Generator(device="cpu").manual_seed(int(seed))
    q = torch.randn(shape, generator=g, dtype=torch.float32) * scale_inputs
    k = torch.randn(shape, generator=g, dtype=torch.float32) * scale_inputs
    v = torch.randn(shape, generator=g, dtype=torch.float32) * scale_inputs
    if outlier_frac > 0.0:
        g2 = torch.Generator(device="cpu").manual_seed(int(outlier_seed if outlier_seed is not None else seed + 1))
        n = k.numel()
        count = int(round(n * outlier_frac))
        idx = torch.randperm(n, generator=g2)[:count]
        flat = k.reshape(-1)
        flat[idx] = flat[idx] * outlier_gain
    return q.to(tdt), k.to(tdt), v.to(tdt)


def to_bits(t) -> np.ndarray:
    """torch fp16/bf16 CPU tensor -> uint16 numpy bit patterns."""
    import torch

    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# --------------------------------------------------------------------------- measurement

def attention_forward_flops(*, b: int, h: int, s: int, d: int, causal: bool) -> float:
    """Work of one forward as the north star counts it: 4*B*H*S^2*D, halved when causal."""
    f = 4.0 * b * h * s * s * d
    return f / 2.0 if causal else f


def reference_forward_flops(*, b: int, h: int, s: int, d: int, causal: bool) -> float:
    """The reference harness's count (run_study.py:95-112): causal is 2*B*H*S*(S+1)*D."""
    if causal:
        return 2.0 * b * h * s * (s + 1) * d
    return 4.0 * b * h * s * s * d


def approximate_bytes(*, b: int, h: int, s: int, d: int, bytes_per_elem: int) -> float:
    """Algorithmic HBM bytes: read q, k, v and write o once (run_study.py:146)."""
    return 4.0 * b * h * s * d * bytes_per_elem


def p95(values) -> float:
    """95th percentile as run_study.py:30-45 takes it (quantiles n=20, index 18)."""
    vals = list(values)
    if not vals:
        raise ValueError("values must not be empty")
    if len(vals) == 1:
        return vals[0]
    return statistics.quantiles(vals, n=20)[18]
