"""Pins of the CPU oracle (oracle/), all on the CPU.

What pins what:

* ``explicit_f32`` (the north-star oracle):
  - against ``explicit_f64`` (same algorithm, another precision),
  - against ``torch.nn.functional.scaled_dot_product_attention`` in fp32 on the CPU
    (a library routine),
  - against a pure-Python brute force on tiny inputs,
  - against known answers (causal row 0 = v0, zero keys -> (prefix) mean, constant v,
    one dominant key, key permutation invariance, head independence, custom scale),
  - against the committed golden fixtures (bit-exact, the oracle is deterministic).
* ``flash_tiled`` (the reference kernel's algorithm, flash_fwd.py:301-446): against the
  explicit oracle within the input dtype's rounding, tile-size independence, and the
  rounding helpers against torch's fp32 -> fp16/bf16 conversions.
* ``eager.eager_attention`` (timed CPU baseline, run_study.py:304-335): in fp32 it must
  equal the explicit oracle; in fp16 it must stay within fp16 rounding of it.
* Planted mistakes: numpy attention variants with a typical bug each (transposed K, no
  scale, causal mask shifted by one, softmax over the wrong axis, V rows misaligned) must
  fail at least one of the checks above.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import eager
from oracle import oracle as O
from tests.golden.fixtures import load_fixture


def _bits(*ts):
    return [O.to_bits(t) for t in ts]


def _ref_np(q, k, v, *, causal, scale=None, bug=None):
    """float64 numpy attention with an optional planted bug (for the mistake tests)."""
    q = q.astype(np.float64); k = k.astype(np.float64); v = v.astype(np.float64)
    d = q.shape[-1]
    sc = 1.0 / math.sqrt(d) if scale is None else scale
    if bug == "no_scale":
        sc = 1.0
    kk = np.swapaxes(k, -1, -2) if bug == "transposed_k" else k  # needs S == D
    s = q @ np.swapaxes(kk, -1, -2) * sc
    if causal:
        n = s.shape[-1]
        off = 1 if bug != "mask_off_by_one" else 0
        mask = np.triu(np.ones((n, n), dtype=bool), off)
        s = np.where(mask, -np.inf, s)
    axis = -1 if bug != "softmax_axis" else -2
    with np.errstate(invalid="ignore"):  # a fully masked row (shifted mask) gives NaN
        s = s - s.max(axis=axis, keepdims=True)
        p = np.exp(s)
        p = p / p.sum(axis=axis, keepdims=True)
    vv = v if bug != "v_shift" else np.roll(v, 1, axis=-2)
    return p @ vv


# ---------------------------------------------------------------- explicit oracle

@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("causal", [False, True])
def test_explicit_f32_vs_f64(dtype, causal):
    q, k, v = O.make_inputs((2, 3, 97, 64), dtype, 1)
    qb, kb, vb = _bits(q, k, v)
    dc = O.dtype_code(dtype)
    o32 = O.explicit_f32(qb, kb, vb, dc, causal=causal)
    o64 = O.explicit_f64(qb, kb, vb, dc, causal=causal)
    assert np.abs(o32 - o64).max() < 2e-6


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(1, 2, 64, 64), (2, 2, 130, 128), (1, 1, 1, 64), (1, 1, 5, 96)])
def test_explicit_vs_torch_sdpa_fp32(dtype, causal, shape):
    q, k, v = O.make_inputs(shape, dtype, 3)
    qb, kb, vb = _bits(q, k, v)
    ours = O.explicit_f32(qb, kb, vb, O.dtype_code(dtype), causal=causal)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=causal)
    assert np.abs(ours - ref.numpy()).max() < 3e-6


def test_explicit_vs_brute_force_python():
    q, k, v = O.make_inputs((1, 1, 5, 3), "float16", 11)
    qf, kf, vf = (t.float().numpy()[0, 0].tolist() for t in (q, k, v))
    for causal in (False, True):
        ours = O.explicit_f32(*_bits(q, k, v), O.FP16, causal=causal)[0, 0]
        for i in range(5):
            js = range(i + 1) if causal else range(5)
            s = [sum(qf[i][t] * kf[j][t] for t in range(3)) / math.sqrt(3) for j in js]
            m = max(s)
            e = [math.exp(x - m) for x in s]
            z = sum(e)
            for t in range(3):
                want = sum(e[n] * vf[j][t] for n, j in enumerate(js)) / z
                assert abs(ours[i][t] - want) < 1e-6


def test_explicit_custom_scale_and_rows_subset():
    q, k, v = O.make_inputs((1, 2, 300, 64), "bfloat16", 5)
    qb, kb, vb = _bits(q, k, v)
    full = O.explicit_f32(qb, kb, vb, O.BF16, causal=True, scale=0.3)
    rows = np.array([0, 7, 150, 299])
    part = O.explicit_f32(qb, kb, vb, O.BF16, causal=True, scale=0.3, rows=rows)
    assert np.array_equal(full[:, :, rows, :], part)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True, scale=0.3)
    assert np.abs(full - ref.numpy()).max() < 3e-6


# ---------------------------------------------------------------- known answers

def test_kat_causal_row0_is_v0():
    q, k, v = O.make_inputs((2, 2, 50, 128), "bfloat16", 2)
    o = O.explicit_f32(*_bits(q, k, v), O.BF16, causal=True)
    assert np.array_equal(o[:, :, 0, :], v.float().numpy()[:, :, 0, :])


def test_kat_zero_keys_prefix_mean():
    q, _, v = O.make_inputs((1, 2, 40, 64), "float16", 4)
    k = torch.zeros_like(q)
    vf = v.float().numpy()
    oc = O.explicit_f32(*_bits(q, k, v), O.FP16, causal=True)
    want = np.cumsum(vf, axis=2) / np.arange(1, 41).reshape(1, 1, -1, 1)
    assert np.abs(oc - want).max() < 1e-5
    on = O.explicit_f32(*_bits(q, k, v), O.FP16, causal=False)
    assert np.abs(on - vf.mean(axis=2, keepdims=True)).max() < 1e-5


def test_kat_constant_values():
    q, k, _ = O.make_inputs((1, 2, 33, 64), "bfloat16", 6)
    v = torch.full(q.shape, -1.25, dtype=torch.bfloat16)
    for causal in (False, True):
        o = O.explicit_f32(*_bits(q, k, v), O.BF16, causal=causal)
        assert np.abs(o + 1.25).max() < 1e-6


def test_kat_dominant_key():
    q, k, v = O.make_inputs((1, 1, 16, 64), "float16", 7)
    q = torch.zeros_like(q)
    q[..., 0] = 8.0
    k = torch.zeros_like(k)
    k[0, 0, 5, 0] = 8.0  # score 64 / sqrt(64) = 8 for key 5, 0 for the rest
    o = O.explicit_f32(*_bits(q, k, v), O.FP16, causal=False)
    w = math.exp(8.0) / (math.exp(8.0) + 15)
    want = w * v.float().numpy()[0, 0, 5] + (1 - w) * (v.float().numpy()[0, 0].sum(0) - v.float().numpy()[0, 0, 5]) / 15
    assert np.abs(o[0, 0] - want).max() < 1e-5


def test_kat_permutation_and_head_independence():
    q, k, v = O.make_inputs((2, 3, 70, 64), "bfloat16", 8)
    perm = torch.randperm(70, generator=torch.Generator().manual_seed(0))
    a = O.explicit_f32(*_bits(q, k, v), O.BF16, causal=False)
    b = O.explicit_f32(*_bits(q, k[:, :, perm], v[:, :, perm]), O.BF16, causal=False)
    assert np.abs(a - b).max() < 1e-6
    one = O.explicit_f32(*_bits(q[1:2, 2:3], k[1:2, 2:3], v[1:2, 2:3]), O.BF16, causal=True)
    full = O.explicit_f32(*_bits(q, k, v), O.BF16, causal=True)
    assert np.array_equal(full[1:2, 2:3], one)


# ---------------------------------------------------------------- golden fixtures

@pytest.mark.parametrize("name", ["c1", "tail_bf16", "tail_fp16"])
def test_golden_fixtures_reproduce(name):
    fx = load_fixture(name)
    dc = O.dtype_code(fx["dtype"])
    o32 = O.explicit_f32(fx["q_bits"], fx["k_bits"], fx["v_bits"], dc, causal=fx["causal"])
    o64 = O.explicit_f64(fx["q_bits"], fx["k_bits"], fx["v_bits"], dc, causal=fx["causal"])
    assert np.array_equal(o32, fx["out_f32"])
    assert np.array_equal(o64, fx["out_f64"])
    # and the inputs are what the seeded generator produces
    q, k, v = O.make_inputs(fx["q_bits"].shape, fx["dtype"], fx["seed"])
    assert np.array_equal(O.to_bits(q), fx["q_bits"])


# ---------------------------------------------------------------- tiled restatement

@pytest.mark.parametrize("dtype,tol", [("float16", 2e-3), ("bfloat16", 1e-2)])
@pytest.mark.parametrize("causal", [False, True])
def test_tiled_fp32acc_vs_explicit(dtype, tol, causal):
    q, k, v = O.make_inputs((1, 4, 200, 64), dtype, 21)
    qb, kb, vb = _bits(q, k, v)
    dc = O.dtype_code(dtype)
    ref = O.explicit_f32(qb, kb, vb, dc, causal=causal)
    for tm, tn in ((64, 64), (128, 64), (64, 128)):
        t = O.upcast(O.flash_tiled(qb, kb, vb, dc, causal=causal, tile_m=tm, tile_n=tn), dc)
        assert np.abs(t - ref).max() <= tol


def test_tiled_input_dtype_accumulation_is_looser_but_bounded():
    q, k, v = O.make_inputs((1, 4, 300, 128), "bfloat16", 22)
    qb, kb, vb = _bits(q, k, v)
    ref = O.explicit_f32(qb, kb, vb, O.BF16, causal=True)
    t32 = O.upcast(O.flash_tiled(qb, kb, vb, O.BF16, causal=True), O.BF16)
    tlp = O.upcast(O.flash_tiled(qb, kb, vb, O.BF16, causal=True, accum_lowp=True), O.BF16)
    e32, elp = np.abs(t32 - ref).max(), np.abs(tlp - ref).max()
    assert e32 <= 1e-2 and elp <= 2.5e-2 and elp >= e32


def test_tiled_l_rounded_option_changes_only_normalisation():
    q, k, v = O.make_inputs((1, 2, 128, 64), "float16", 23)
    qb, kb, vb = _bits(q, k, v)
    a = O.upcast(O.flash_tiled(qb, kb, vb, O.FP16, causal=True), O.FP16)
    b = O.upcast(O.flash_tiled(qb, kb, vb, O.FP16, causal=True, l_rounded=True), O.FP16)
    assert np.abs(a - b).max() < 2e-3


def test_rounding_matches_torch_conversions():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10,
        rng.standard_normal(2000).astype(np.float32) * 1e-6,      # fp16 subnormals
        np.array([65504, 65519, 65520, 1e6, -1e6, 6.1e-5, 5.96e-8, 2.98e-8, 0.0, -0.0], np.float32),
        (1 + np.arange(1, 400) * 2.0 ** -11).astype(np.float32),  # fp16 ties
        (1 + np.arange(1, 400) * 2.0 ** -8).astype(np.float32),   # bf16 ties
    ])
    t = torch.from_numpy(x)
    assert np.array_equal(O.round_to(x, O.FP16), t.to(torch.float16).view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(O.round_to(x, O.BF16), t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    h = t.to(torch.float16)
    assert np.array_equal(O.upcast(O.to_bits(h), O.FP16), h.float().numpy())


# ---------------------------------------------------------------- eager restatement (CPU baseline)

def test_eager_fp32_equals_oracle_and_fp16_is_close():
    q, k, v = O.make_inputs((1, 2, 96, 64), "float16", 30)
    ref = O.explicit_f32(*_bits(q, k, v), O.FP16, causal=True)
    e32 = eager.eager_attention(q.float(), k.float(), v.float(), causal=True).numpy()
    assert np.abs(e32 - ref).max() < 3e-6
    e16 = eager.eager_attention(q, k, v, causal=True).float().numpy()
    assert np.abs(e16 - ref).max() < 1e-2
    per = eager.eager_attention_per_head(q, k, v, causal=True)
    assert np.abs(torch.cat(per, dim=1).float().numpy() - e16).max() == 0


# ---------------------------------------------------------------- measurement helpers

def test_flop_and_byte_formulas():
    assert O.attention_forward_flops(b=1, h=8, s=8192, d=128, causal=True) == 2 * 8 * 8192 ** 2 * 128
    assert O.attention_forward_flops(b=4, h=16, s=4096, d=64, causal=False) == 4 * 4 * 16 * 4096 ** 2 * 64
    assert O.reference_forward_flops(b=1, h=8, s=512, d=128, causal=True) == 2 * 8 * 512 * 513 * 128
    assert O.approximate_bytes(b=1, h=8, s=8192, d=128, bytes_per_elem=2) == 4 * 8 * 8192 * 128 * 2
    assert O.p95([5.0]) == 5.0
    assert O.p95(list(range(1, 21))) == pytest.approx(19.95)


def test_inputs_are_seeded_and_outliers_counted():
    a = O.make_inputs((1, 2, 64, 64), "bfloat16", 9)
    b = O.make_inputs((1, 2, 64, 64), "bfloat16", 9)
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    base = O.make_inputs((1, 2, 100, 64), "float16", 9)
    out = O.make_inputs((1, 2, 100, 64), "float16", 9, outlier_frac=0.01, outlier_seed=10)
    changed = (out[1] != base[1]).sum().item()
    assert 0 < changed <= round(base[1].numel() * 0.01)
    assert torch.equal(out[0], base[0]) and torch.equal(out[2], base[2])


# ---------------------------------------------------------------- planted mistakes

@pytest.mark.parametrize("bug", ["no_scale", "transposed_k", "mask_off_by_one", "softmax_axis", "v_shift"])
def test_planted_mistakes_are_caught(bug):
    """A buggy restatement must fail at least one of the checks that pin the oracle."""
    q, k, v = O.make_inputs((1, 2, 64, 64), "float16", 0)
    qf, kf, vf = (t.float().numpy() for t in (q, k, v))
    failures = 0
    for causal in (False, True):
        good = _ref_np(qf, kf, vf, causal=causal)
        bad = _ref_np(qf, kf, vf, causal=causal, bug=bug)
        lib = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=causal).numpy()
        assert np.abs(good - lib).max() < 1e-5  # the check itself accepts the correct one
        failures += int(np.abs(bad - lib).max() > 1e-3)
        if causal:
            failures += int(not np.allclose(bad[:, :, 0, :], vf[:, :, 0, :]))
    assert failures > 0
