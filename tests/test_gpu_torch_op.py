"""The custom operator on the GPU: opcheck, compiled graphs and eager agree with sdpa."""

from __future__ import annotations

import pytest

from tests.parity_util import as_f32, check_close, inputs, oracle_f32, say

pytestmark = pytest.mark.gpu


def test_opcheck(gpu):
    import torch

    from tiledattention import torch_op  # noqa: F401

    q, k, v = (t.cuda() for t in inputs((1, 2, 128, 64), "float16", 21))
    say("torch.library.opcheck tiledattention::sdpa_fwd (1,2,128,64) fp16")
    torch.library.opcheck(torch.ops.tiledattention.sdpa_fwd.default, (q, k, v, True, None),
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.parametrize("d", [64, 100])
def test_compiled_graph_matches_eager(gpu, d):
    import torch

    from tiledattention import sdpa, torch_op  # noqa: F401

    qc, kc, vc = inputs((1, 2, 192, d), "bfloat16", 22 + d)
    q, k, v = (t.cuda() for t in (qc, kc, vc))

    def fn(q, k, v):
        return torch.ops.tiledattention.sdpa_fwd(q, k, v, True, None)

    say(f"torch.compile(aot_eager, fullgraph) over the operator, D={d}")
    compiled = torch.compile(fn, backend="aot_eager", fullgraph=True)
    got = compiled(q, k, v)
    torch.cuda.synchronize()
    assert got.is_contiguous() and got.shape == q.shape
    ref = sdpa(q, k, v, causal=True)
    assert bool((got == ref).all())
    check_close(as_f32(got), oracle_f32(qc, kc, vc, causal=True), "bfloat16", what=f"op D={d}")


@pytest.mark.parametrize("tm,tn,acc", [(64, 128, 0), (128, 64, 1), (64, 64, 1)])
def test_explicit_tile_and_accum_match_the_knobs(gpu, monkeypatch, tm, tn, acc):
    """The operator's tile/accum arguments select the same kernel the env knobs select: the
    outputs are bit-identical, and both meet the oracle bound (input-dtype accumulation at
    its looser bound)."""
    import torch

    from tiledattention import sdpa, torch_op  # noqa: F401
    from tests.parity_util import LOWP_TOL

    qc, kc, vc = inputs((1, 2, 320, 128), "float16", 31 + tm + tn + acc)
    q, k, v = (t.cuda() for t in (qc, kc, vc))
    say(f"operator tile=({tm},{tn}) accum={acc} vs knobs")
    got = torch.ops.tiledattention.sdpa_fwd(q, k, v, False, None, tm, tn, acc)
    monkeypatch.setenv("TILEDATTN_TILE_M", str(tm))
    monkeypatch.setenv("TILEDATTN_TILE_N", str(tn))
    monkeypatch.setenv("TILEDATTN_ACCUM_MODE", "fp16" if acc else "fp32")
    ref = sdpa(q, k, v, causal=False)
    torch.cuda.synchronize()
    assert bool((got == ref).all())
    check_close(as_f32(got), oracle_f32(qc, kc, vc, causal=False), "float16", what="op tile",
                tol=LOWP_TOL["float16"] if acc else None)
