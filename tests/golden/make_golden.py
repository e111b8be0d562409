"""Writes the committed golden fixtures in this directory.

Each fixture holds seeded inputs (fp16/bf16 bit patterns) and the explicit fp32 and fp64
oracle outputs, computed by this repository's oracle (oracle/attention_oracle.c).  The
reference holds no numeric fixtures of its own for this path (its only numeric check,
tests/test_sdpa_correctness_small.py, draws inputs on the GPU at run time), so these pin
the oracle's outputs against silent change and carry them to the GPU box.

Run from the repository root: ``python -m tests.golden.make_golden``.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402

HERE = Path(__file__).resolve().parent

CASES = {
    # C1: the reference's example.py:19-24 workload, inputs from the CPU generator.
    "c1": dict(shape=(1, 2, 64, 64), dtype="float16", seed=0, causal=True),
    # ragged tail, bf16, D=128
    "tail_bf16": dict(shape=(1, 2, 100, 128), dtype="bfloat16", seed=42, causal=True),
    # ragged tail, fp16, D=64, non-causal
    "tail_fp16": dict(shape=(2, 1, 77, 64), dtype="float16", seed=43, causal=False),
}


def make(name: str, shape, dtype: str, seed: int, causal: bool) -> Path:
    q, k, v = O.make_inputs(shape, dtype, seed)
    dc = O.dtype_code(dtype)
    qb, kb, vb = O.to_bits(q), O.to_bits(k), O.to_bits(v)
    out32 = O.explicit_f32(qb, kb, vb, dc, causal=causal)
    out64 = O.explicit_f64(qb, kb, vb, dc, causal=causal)
    path = HERE / f"{name}.npz"
    np.savez_compressed(path, q=qb, k=kb, v=vb, out_f32=out32, out_f64=out64,
                        dtype=np.array(dtype), causal=np.array(causal), seed=np.array(seed))
    return path


def main() -> None:
    for name, cfg in CASES.items():
        p = make(name, **cfg)
        print(f"wrote {p} ({p.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
