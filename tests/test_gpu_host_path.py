"""GPU checks of the host launch path: cached launch plans follow knob changes and cache
resets, inputs the kernel cannot read in place (misaligned, strided) are copied, and the
output matches the oracle in every case.  Every case names itself before touching the GPU."""

from __future__ import annotations

import pytest

from tests.parity_util import as_f32, check_close, inputs, knobs, oracle_f32, say

pytestmark = pytest.mark.gpu


def _sdpa(q, k, v, **kw):
    import torch

    from tiledattention_amd import sdpa

    out = sdpa(q, k, v, **kw)
    torch.cuda.synchronize()
    return out


def test_knob_changes_between_calls_take_effect(gpu):
    import torch

    from tiledattention_amd.kernels import compile_cache as cc

    q, k, v = inputs((1, 2, 384, 64), "float16", 21)
    ref = oracle_f32(q, k, v, causal=True)
    dev = torch.device("cuda:0")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    cc.reset_cache_for_tests()
    seen = []
    for tiles in ((64, 64), (128, 128), (64, 64), (None, None)):
        say(f"host path fp16 (1,2,384,64) causal tiles={tiles}")
        env = {"tile_m": tiles[0], "tile_n": tiles[1]}
        with knobs(**env):
            out = _sdpa(qd, kd, vd, causal=True)
        check_close(as_f32(out), ref, "float16", what=f"tiles={tiles}")
        seen.append(cc.cache_size())
    # (64,64) and (128,128) each add a kernel; repeating (64,64) reuses it; default adds one
    assert seen == [1, 2, 2, 3], seen
    say("host path: invalid sync mode raises on every call")
    for _ in range(2):
        with knobs(sync_mode="sometimes"), pytest.raises(ValueError, match="TILEDATTN_SYNC_MODE"):
            _sdpa(qd, kd, vd, causal=True)
    say("host path: a cache reset is seen by the next call")
    cc.reset_cache_for_tests()
    out = _sdpa(qd, kd, vd, causal=True)
    assert cc.cache_size() == 1
    check_close(as_f32(out), ref, "float16", what="after reset")


def test_misaligned_and_strided_inputs(gpu):
    """A dense view at a 2-byte offset (the kernel needs 16-byte aligned rows) and a view
    whose row stride is not a multiple of 8 elements are copied; a [B,S,H,D] view is read
    in place."""
    import torch

    q, k, v = inputs((1, 2, 256, 128), "bfloat16", 5)
    ref = oracle_f32(q, k, v, causal=False)
    dev = torch.device("cuda:0")
    flat = [torch.empty(t.numel() + 1, dtype=t.dtype, device=dev) for t in (q, k, v)]
    mis = []
    for buf, t in zip(flat, (q, k, v)):
        view = buf[1:].view(t.shape)
        view.copy_(t.to(dev))
        assert view.is_contiguous() and view.data_ptr() % 16 != 0
        mis.append(view)
    say("host path bf16 (1,2,256,128) misaligned dense views")
    check_close(as_f32(_sdpa(*mis, causal=False)), ref, "bfloat16", what="misaligned")
    wide = [torch.zeros(1, 2, 256, 132, dtype=t.dtype, device=dev) for t in (q, k, v)]
    odd = []
    for w, t in zip(wide, (q, k, v)):
        w[..., :128].copy_(t.to(dev))
        odd.append(w[..., :128])
    say("host path bf16 (1,2,256,128) row stride 132")
    check_close(as_f32(_sdpa(*odd, causal=False)), ref, "bfloat16", what="row stride 132")
    bshd = [t.transpose(1, 2).contiguous().to(dev).transpose(1, 2) for t in (q, k, v)]
    say("host path bf16 (1,2,256,128) [B,S,H,D] views")
    check_close(as_f32(_sdpa(*bshd, causal=False)), ref, "bfloat16", what="BSHD views")
    # the same shapes again: cached plans, same answers
    say("host path bf16 repeated calls on cached plans")
    check_close(as_f32(_sdpa(*mis, causal=False)), ref, "bfloat16", what="misaligned again")
    check_close(as_f32(_sdpa(*bshd, causal=False)), ref, "bfloat16", what="BSHD again")
