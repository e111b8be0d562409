"""Causal query-block pairs on the eight-wave kernel (one workgroup runs blocks nq - 1 - j and
j of a head, ``ta_fwd_args.sched`` 1 on grids of two or more workgroups per CU, or 3).

Each block is computed exactly as in the one-block-per-workgroup grid, so the paired output
must equal the unpaired one (TILEDATTN_SCHED=0) bit for bit, and meet the north-star bound
against the fp32 oracle (sampled rows for the long sequences).  Every case names itself."""

from __future__ import annotations

import pytest

from tests.parity_util import as_f32, check_close, inputs, knobs, oracle_f32, sample_rows, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,dtype,sched", [
    ((1, 8, 8192, 128), "bfloat16", None),   # C3 at S=8192: 512 blocks, pairs by default
    ((2, 8, 4096, 64), "float16", None),     # D = 64 causal, 512 blocks
    ((1, 16, 4200, 128), "bfloat16", None),  # odd block count (33): the middle block alone; tail
    ((1, 8, 8192, 160), "bfloat16", "3"),    # D = 160: never paired (sched 3 has no effect)
    ((1, 2, 1000, 128), "float16", "3"),     # forced on a small grid, ragged tail
    ((1, 1, 300, 64), "bfloat16", "3"),      # nq = 3
])
def test_pairs_match_unpaired_and_oracle(gpu, shape, dtype, sched):
    import torch

    q, k, v = inputs(shape, dtype, 70 + shape[2] % 97)
    dev = torch.device("cuda:0")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    from tiledattention import sdpa

    say(f"pairs {dtype} {shape} causal sched={sched or 'default'}")
    with knobs(sched=sched):
        got = sdpa(qd, kd, vd, causal=True)
    say(f"unpaired {dtype} {shape} causal sched=0")
    with knobs(sched="0"):
        ref_gpu = sdpa(qd, kd, vd, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(got, ref_gpu), float((got.float() - ref_gpu.float()).abs().max())
    rows = sample_rows(shape[2], 96) if shape[2] >= 4096 else None
    check_close(as_f32(got, rows), oracle_f32(q, k, v, causal=True, rows=rows), dtype, what=f"pairs {shape}")
