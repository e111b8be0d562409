"""The wide kernel (``ta_fwd_wide_*``: 32 query rows a workgroup, its eight waves splitting
the keys of every pass; the 64-row fp32 tiles on grids of one round of the CUs) against the
CPU oracle.

Cases cover one, two and four passes of keys (512 keys a pass at D = 128, 1024 at D = 64),
causal and not, ragged S (rows and keys past S: the tail variants, including S a multiple of
32 but not of a wave's 64 keys), both dtypes and head dims, head dims padded in place
(d_real), strided views and a custom scale.  Each case first checks that the library
describes the wide kernel for it (``ta_describe_launch``), names itself before touching the
GPU, and compares the whole output at the north-star bound.
"""

from __future__ import annotations

import random

import pytest

from tests.parity_util import as_f32, check_close, inputs, kernel_for, oracle_f32, run_gpu, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,dtype,causal", [
    ((1, 8, 512, 128), "bfloat16", True),    # C3 S=512: one pass
    ((1, 8, 1024, 128), "bfloat16", True),   # C3 S=1024: two passes
    ((1, 8, 1024, 64), "float16", False),    # C2's shape: one pass of 1024 keys
    ((1, 4, 2048, 64), "bfloat16", True),    # two passes at D = 64
    ((1, 3, 2048, 128), "float16", True),    # four passes on 192 blocks
    ((1, 4, 300, 128), "bfloat16", True),    # ragged: rows and keys past S
    ((1, 4, 300, 64), "float16", False),
    ((2, 3, 544, 128), "bfloat16", False),   # a multiple of 32, not of 64: tail variant
    ((1, 5, 1000, 128), "float16", False),   # two passes, ragged
    ((1, 2, 64, 64), "float16", True),       # C1
    ((3, 2, 96, 64), "bfloat16", True),
    ((1, 1, 1, 128), "float16", True),       # one row
])
def test_wide_matches_oracle(gpu, shape, dtype, causal):
    q, k, v = inputs(shape, dtype, 500 + shape[2] % 89)
    kernel = kernel_for(q, k, v, causal=causal)
    assert kernel.startswith("ta_fwd_wide_"), kernel
    say(f"wide {kernel} {dtype} {shape} causal={causal}")
    out = run_gpu(q, k, v, causal=causal)
    assert out.shape == q.shape and out.dtype == q.dtype
    check_close(as_f32(out), oracle_f32(q, k, v, causal=causal), dtype, what=f"wide {shape} causal={causal}")


@pytest.mark.parametrize("shape,dtype,causal", [
    ((1, 4, 512, 112), "bfloat16", True),   # kernel D = 128, columns 112.. zero, not written
    ((1, 4, 700, 40), "float16", False),    # kernel D = 64, 40 columns
])
def test_wide_head_dims_padded_in_place(gpu, shape, dtype, causal):
    q, k, v = inputs(shape, dtype, 77)
    kernel = kernel_for(q, k, v, causal=causal)
    assert kernel.startswith("ta_fwd_wide_"), kernel
    say(f"wide padded head dim {kernel} {dtype} {shape} causal={causal}")
    out = run_gpu(q, k, v, causal=causal)
    assert out.shape == q.shape
    check_close(as_f32(out), oracle_f32(q, k, v, causal=causal), dtype, what=f"wide padded {shape}")


def test_wide_strided_views_custom_scale_and_repeat(gpu):
    """q, k, v as [B, H, S, D] views of [B, S, H, D] storage (row stride H * D), scale 0.3,
    and a second call that must give the same bits."""
    import torch

    from tiledattention import sdpa

    shape = (1, 6, 640, 128)
    q, k, v = inputs(shape, "bfloat16", 31)
    dev = torch.device("cuda:0")
    qs, ks, vs = (t.transpose(1, 2).contiguous().to(dev).transpose(1, 2) for t in (q, k, v))
    assert qs.stride(2) == shape[1] * shape[3]
    kernel = kernel_for(qs, ks, vs, causal=True)
    assert kernel.startswith("ta_fwd_wide_"), kernel
    say(f"wide strided views scale=0.3 {kernel} {shape}")
    out1 = sdpa(qs, ks, vs, causal=True, scale=0.3)
    out2 = sdpa(qs, ks, vs, causal=True, scale=0.3)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    check_close(as_f32(out1), oracle_f32(q, k, v, causal=True, scale=0.3), "bfloat16", what="wide strided")


def _wide_draw(rng) -> dict:
    """A configuration inside the wide kernel's rule at 256 CUs: S <= 1024, B * H * ceil(S/32)
    <= 256; head dims that reach kernel D = 64 or 128 (in place, or padded on the host for
    33 and 100), never (64, 96] (the native D = 96 kernel)."""
    s = rng.choice([1, 31, 33, 64, 200, 255, 256, 257, 500, 511, 640, 777, 1000, 1024])
    blocks = -(-s // 32)
    bh_max = max(1, 256 // blocks)
    bh = rng.randint(1, min(bh_max, 12))
    b = rng.choice([d for d in (1, 2, 3) if bh % d == 0])
    return dict(b=b, h=bh // b, s=s, d=rng.choice([8, 24, 33, 40, 56, 64, 100, 104, 120, 128]),
                dtype=rng.choice(["float16", "bfloat16"]), causal=rng.random() < 0.5,
                scale=rng.choice([None, None, 0.05, 0.3]), mag=rng.choice([0.5, 1.0, 2.0]),
                bshd=rng.random() < 0.3, seed=rng.randrange(1 << 30))


_WIDE_CASES = [_wide_draw(r) for r in [random.Random(20261202)] for _ in range(24)]


@pytest.mark.parametrize("case", _WIDE_CASES, ids=[f"w{i}" for i in range(len(_WIDE_CASES))])
def test_wide_randomized(gpu, case):
    """Seeded random configurations inside the wide rule against the explicit fp32 oracle, at
    the north-star tolerance scaled by the input magnitude; draws with a sharp softmax
    (logit spread above 6) at the P-rounding bound 3 u max|v| instead (the reasoning of
    tests/test_gpu_randomized.py)."""
    import math

    import numpy as np
    import torch

    from tiledattention import sdpa
    from tests.parity_util import TOL

    c = case
    q, k, v = inputs((c["b"], c["h"], c["s"], c["d"]), c["dtype"], c["seed"], scale_inputs=c["mag"])
    dev = torch.device("cuda:0")
    if c["bshd"]:
        qd, kd, vd = (t.transpose(1, 2).contiguous().to(dev).transpose(1, 2) for t in (q, k, v))
    else:
        qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    kernel = kernel_for(qd, kd, vd, causal=c["causal"])
    assert kernel.startswith("ta_fwd_wide_"), (kernel, c)
    say(f"wide random {kernel} {c}")
    out = sdpa(qd, kd, vd, causal=c["causal"], scale=c["scale"])
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == q.dtype
    scale = c["scale"] if c["scale"] is not None else 1.0 / math.sqrt(c["d"])
    spread = scale * c["mag"] ** 2 * math.sqrt(c["d"])
    tol = TOL[c["dtype"]] * max(1.0, c["mag"])
    if spread > 6.0:
        u = 2.0 ** -8 if c["dtype"] == "bfloat16" else 2.0 ** -11
        tol = max(tol, 3 * u * float(np.abs(v.float().numpy()).max()))
    ref = oracle_f32(q, k, v, causal=c["causal"], scale=c["scale"])
    check_close(as_f32(out), ref, c["dtype"], tol=tol, what=f"wide random (logit spread {spread:.1f})")
