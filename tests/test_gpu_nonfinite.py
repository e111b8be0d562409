"""Non-finite inputs on the GPU: NaN and inf propagate to exactly the output elements the
oracle's explicit softmax(Q K^T * scale + mask) V makes non-finite, on the whole-row and
the split-key-range paths; every finite element stays within tolerance.

IEEE rules fix the expectations: a NaN score makes its row's max, exponent and sum NaN; a
causally masked score is replaced by -inf whatever its value, so rows before a NaN key stay
finite.  One case is implementation-defined: a NaN in a value row j under the causal mask.
The oracle computes row i over its visible keys only (rows i >= j are NaN); a tiled kernel
multiplies the masked keys' P = 0 by V inside the diagonal tile, and 0 x NaN = NaN, so here
every row of the query block holding j is NaN as well, from the block's first row on (128
rows for the 128-row and 64-row kernels, whose diagonal key step is 128 keys; 32 for the
wide kernel's blocks; the reference's tiled kernel does the same at its own tile size; its
eager baseline, which multiplies the full masked P, makes every row NaN).  That case is
checked against exactly that rule, with the block size of the kernel that ran."""

from __future__ import annotations

import numpy as np
import pytest

from tests.parity_util import TOL, as_f32, inputs, kernel_for, oracle_f32, run_gpu, say

pytestmark = pytest.mark.gpu


def _poison(t, row, value):
    t = t.clone()
    t[0, 1, row, :] = value
    return t


def _compare(got: np.ndarray, ref: np.ndarray, dtype: str, what: str, nan_from_row=None):
    nan_g, nan_r = np.isnan(got), np.isnan(ref)
    if nan_from_row is not None:
        # rows of the poisoned head from nan_from_row on are NaN in full; the oracle's own
        # NaN rows lie among them
        assert not nan_r[0, 1, :nan_from_row, :].any()
        nan_r = nan_r.copy()
        nan_r[0, 1, nan_from_row:, :] = True
        ref = np.where(nan_r, np.nan, ref)
    assert (nan_g == nan_r).all(), f"{what}: NaN positions differ ({nan_g.sum()} vs {nan_r.sum()})"
    fin = np.isfinite(ref)
    assert (np.isfinite(got) == fin).all(), f"{what}: finite positions differ"
    err = float(np.abs(got[fin].astype(np.float64) - ref[fin]).max()) if fin.any() else 0.0
    print(f"[check] {what} non-finite={int((~fin).sum())} max_abs_err={err:.3e}", flush=True)
    assert err <= TOL[dtype], f"{what}: {err}"


@pytest.mark.parametrize("tensor,row,value", [
    ("q", 37, float("nan")), ("k", 300, float("nan")), ("v", 300, float("nan")),
    ("k", 5, float("inf")),
])
@pytest.mark.parametrize("causal", [False, True])
def test_nonfinite_propagation(gpu, tensor, row, value, causal):
    q, k, v = inputs((1, 2, 640, 128), "bfloat16", 99)
    if tensor == "q":
        q = _poison(q, row, value)
    elif tensor == "k":
        k = _poison(k, row, value)
    else:
        v = _poison(v, row, value)
    with np.errstate(invalid="ignore", over="ignore"):
        ref = oracle_f32(q, k, v, causal=causal)
    assert not np.isfinite(ref).all()
    poisoned_v = tensor == "v" and causal
    if poisoned_v:
        assert np.isnan(ref[0, 1, row:, :]).all() and np.isfinite(ref[0, 1, :row, :]).all()
    for split in ("off", 1):
        kernel = kernel_for(q, k, v, causal=causal, split=split, accum_mode="fp32")
        block = 32 if kernel.startswith("ta_fwd_wide_") else 128
        nan_from = (row // block) * block if poisoned_v else None
        say(f"non-finite {tensor}[0,1,{row},:]={value} causal={causal} split={split} kernel={kernel}")
        out = run_gpu(q, k, v, causal=causal, split=split, accum_mode="fp32")
        _compare(as_f32(out), ref, "bfloat16", f"{tensor} row {row} = {value} causal={causal} split={split}",
                 nan_from_row=nan_from)
