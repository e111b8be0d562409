"""The GPU parity helpers' own behaviour, on CPU tensors: a non-finite value anywhere in
the output fails the sampled-row comparison, not only one inside the sampled rows."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.parity_util import as_f32, check_close, sample_rows


def _out():
    g = torch.Generator().manual_seed(3)
    return torch.randn((1, 2, 300, 64), generator=g).to(torch.bfloat16)


def test_sampled_rows_pass_when_every_element_is_finite():
    out = _out()
    rows = sample_rows(300, 8)
    got = as_f32(out, rows)
    assert got.shape == (1, 2, len(rows), 64)
    check_close(got, got.copy(), "bfloat16", what="self")


@pytest.mark.parametrize("value", [float("nan"), float("inf"), -float("inf")])
def test_non_finite_outside_the_sampled_rows_fails(value):
    out = _out()
    rows = sample_rows(300, 8)
    unsampled = int(np.setdiff1d(np.arange(300), rows)[0])
    out[0, 1, unsampled, 5] = value
    with pytest.raises(AssertionError, match="non-finite output elements"):
        as_f32(out, rows)


def test_whole_output_comparison_still_checks_finiteness():
    out = _out()
    out[0, 0, 7, 0] = float("nan")
    got = as_f32(out)  # no rows: check_close asserts on the full array
    with pytest.raises(AssertionError, match="non-finite output"):
        check_close(got, np.zeros_like(got), "bfloat16", what="nan")
