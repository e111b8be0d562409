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


@pytest.mark.parametrize("knobs", [
    {}, {"TILEDATTN_TILE_M": "64", "TILEDATTN_TILE_N": "128"}, {"TILEDATTN_ACCUM_MODE": "fp16"},
    {"TILEDATTN_SPLIT": "2"}, {"TILEDATTN_SPLIT": "pairs"}, {"TILEDATTN_DISABLE_ALIGNED_FASTPATH": "1"},
    {"TILEDATTN_SCHED": "3"}, {"TILEDATTN_SYNC_MODE": "strict"},
])
def test_cpp_operator_equals_sdpa(gpu, monkeypatch, knobs):
    """The C++ operator plans through ta_plan_call and the Python layer through its own
    policy: under every knob setting they launch the same kernel with the same arguments,
    so the outputs are bit-identical, over shapes that take every path (64- and 128-row
    tiles, causal pairs, 256-row blocks, the split, in-kernel and host head-dim padding,
    [B,S,H,D] views)."""
    import torch

    from tiledattention import sdpa, torch_op  # noqa: F401

    for key, val in knobs.items():
        monkeypatch.setenv(key, val)
    shapes = [((1, 8, 1000, 128), True), ((1, 8, 4096, 128), True), ((2, 4, 777, 64), False),
              ((1, 3, 1300, 72), True), ((1, 2, 300, 99), False), ((4, 16, 1024, 128), False),
              ((1, 2, 64, 160), True)]
    for i, (shape, causal) in enumerate(shapes):
        qc, kc, vc = inputs(shape, "bfloat16" if i % 2 else "float16", 300 + i)
        q, k, v = (t.cuda() for t in (qc, kc, vc))
        if i == 2:  # a [B,S,H,D] tensor viewed as [B,H,S,D]
            q, k, v = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v))
        say(f"C++ operator vs sdpa {shape} causal={causal} knobs={knobs}")
        errors = []
        try:
            got = torch.ops.tiledattention.sdpa_fwd(q, k, v, causal, None)
        except (RuntimeError, ValueError) as exc:
            errors.append(exc)
        try:
            ref = sdpa(q, k, v, causal=causal)
        except (RuntimeError, ValueError) as exc:  # the tile knob without a kernel for this D
            errors.append(exc)
        assert len(errors) in (0, 2), errors  # both reject, or both run
        if errors:
            continue
        torch.cuda.synchronize()
        assert got.shape == ref.shape and got.is_contiguous()
        assert torch.equal(got, ref), (shape, float((got.float() - ref.float()).abs().max()))


def test_cpp_operator_errors_and_host_time(gpu, monkeypatch):
    """Checks in the Python layer's order and words; then the host time per call of the C++
    operator against sdpa (printed; the operator saves the ctypes hop and the Python policy
    lookup)."""
    import time

    import torch

    from tiledattention import sdpa, torch_op  # noqa: F401

    q = torch.zeros((1, 2, 64, 64), dtype=torch.float16, device="cuda")
    op = torch.ops.tiledattention.sdpa_fwd
    with pytest.raises(RuntimeError, match="q, k, and v must have identical dtype"):
        op(q, q, q.to(torch.bfloat16), False, None)
    with pytest.raises(RuntimeError, match="scale must be a positive number"):
        op(q, q, q, False, -1.0)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        op(q.cpu(), q, q, False, None)
    with pytest.raises(ValueError, match="Unsupported tile"):
        op(q, q, q, False, None, 32, 64, -1)
    monkeypatch.setenv("TILEDATTN_ACCUM_MODE", "fp8")
    with pytest.raises(ValueError, match="Unsupported TILEDATTN_ACCUM_MODE='fp8'"):
        op(q, q, q, False, None)
    monkeypatch.setenv("TILEDATTN_ACCUM_MODE", "fp32")
    monkeypatch.setenv("TILEDATTN_SPLIT", "x")
    with pytest.raises(ValueError, match="TILEDATTN_SPLIT must be"):
        op(q, q, q, False, None)
    monkeypatch.delenv("TILEDATTN_SPLIT")
    qs = torch.randn((1, 2, 64, 64), dtype=torch.float16, device="cuda")  # a kernel shorter than the host path
    say("host time per call: C++ operator vs sdpa (B1 H2 S64 D64 causal)")
    for fn in (lambda: op(qs, qs, qs, True, None), lambda: sdpa(qs, qs, qs, causal=True)):
        for _ in range(50):
            fn()
        torch.cuda.synchronize()
    res = {}
    for name, fn in (("cpp_op", lambda: op(qs, qs, qs, True, None)), ("sdpa", lambda: sdpa(qs, qs, qs, causal=True))):
        best = float("inf")
        for _ in range(5):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(200):
                fn()
            best = min(best, (time.perf_counter() - t0) / 200)
            torch.cuda.synchronize()
        res[name] = best * 1e6
    print(f"[host] us per call (200 queued calls, best of 5): {res}", flush=True)
    assert res["cpp_op"] > 0 and res["sdpa"] > 0
