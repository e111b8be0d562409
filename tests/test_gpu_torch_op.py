"""The custom operator on the GPU: opcheck, compiled graphs and eager agree with sdpa."""

from __future__ import annotations

import pytest

from tests.parity_util import as_f32, check_close, inputs, oracle_f32, say

pytestmark = pytest.mark.gpu


def test_opcheck(gpu):
    import torch

    from tiledattention_amd import torch_op  # noqa: F401

    q, k, v = (t.cuda() for t in inputs((1, 2, 128, 64), "float16", 21))
    say("torch.library.opcheck tiledattention::sdpa_fwd (1,2,128,64) fp16")
    torch.library.opcheck(torch.ops.tiledattention.sdpa_fwd.default, (q, k, v, True, None),
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.parametrize("d", [64, 100])
def test_compiled_graph_matches_eager(gpu, d):
    import torch

    from tiledattention_amd import sdpa, torch_op  # noqa: F401

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
