"""GPU checks of the host launch path: cached launch plans follow knob changes and cache
resets, inputs the kernel cannot read in place (misaligned, strided) are copied, and the
output matches the oracle in every case.  Every case names itself before touching the GPU."""

from __future__ import annotations

import numpy as np
import pytest

from tests.parity_util import TOL, as_f32, check_close, inputs, knobs, oracle_f32, sample_rows, say

pytestmark = pytest.mark.gpu


def _sdpa(q, k, v, **kw):
    import torch

    from tiledattention import sdpa

    out = sdpa(q, k, v, **kw)
    torch.cuda.synchronize()
    return out


def test_knob_changes_between_calls_take_effect(gpu):
    import torch

    from tiledattention.kernels import compile_cache as cc

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
    # (64,64) and (128,128) each add a kernel; repeating (64,64) reuses it; the default for
    # this grid (2 x 6 blocks of 64 rows, fewer than the CUs) is (64,64) too
    assert seen == [1, 2, 2, 2], seen
    from tiledattention.kernels import flash_fwd as ff
    assert ff._default_tile_config_for_shape_gfx950(seq_len=384, head_dim=64, causal=True, n_bh=2,
                                                    compute_units=256) == (64, 64)
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


def test_expanded_and_overlapping_rows_are_copied(gpu):
    """K and V expanded along S (row stride 0) and a view whose rows overlap (row stride
    below D) cannot be read in place: the host copies them, as the reference copies every
    input (flash_fwd.py:865-867), and the result matches the oracle on the materialised
    tensors."""
    import torch

    dev = torch.device("cuda:0")
    q, k, v = inputs((1, 2, 192, 64), "float16", 41)
    k1 = k[:, :, :1].expand(-1, -1, 192, -1)
    v1 = v[:, :, 5:6].expand(-1, -1, 192, -1)
    ref = oracle_f32(q, k1.contiguous(), v1.contiguous(), causal=True)
    say("host path fp16 (1,2,192,64) k, v expanded along S (row stride 0)")
    kd, vd = k[:, :, :1].to(dev).expand(-1, -1, 192, -1), v[:, :, 5:6].to(dev).expand(-1, -1, 192, -1)
    assert kd.stride(2) == 0 and vd.stride(2) == 0
    out = _sdpa(q.to(dev), kd, vd, causal=True)
    check_close(as_f32(out), ref, "float16", what="expanded k/v")
    # every output row is v[5] (one distinct key value, one distinct value row)
    assert np.allclose(as_f32(out), v[:, :, 5:6].float().numpy(), atol=2e-3)

    base = [torch.empty(2 * 200 * 32 + 64, dtype=torch.float16) for _ in range(3)]
    for i, b in enumerate(base):
        b.copy_(torch.randn(b.numel(), generator=torch.Generator().manual_seed(50 + i)).half())
    views = [b.as_strided((1, 2, 200, 64), (2 * 200 * 32, 200 * 32, 32, 1)) for b in base]
    ref = oracle_f32(*(t.contiguous() for t in views), causal=False)
    say("host path fp16 (1,2,200,64) overlapping rows (row stride 32 < D)")
    dviews = [b.to(dev).as_strided((1, 2, 200, 64), (2 * 200 * 32, 200 * 32, 32, 1)) for b in base]
    check_close(as_f32(_sdpa(*dviews, causal=False)), ref, "float16", what="overlapping rows")


@pytest.mark.parametrize("shape,dtype,causal,tiles", [
    ((1, 2, 1024, 64), "float16", False, None),
    ((1, 2, 2048, 128), "bfloat16", True, None),
    ((1, 2, 1024, 160), "bfloat16", True, None),
    ((1, 2, 512, 128), "float16", False, (64, 64)),
    ((1, 2, 512, 64), "bfloat16", True, (64, 128)),
    ((1, 2, 512, 128), "float16", True, (128, 128)),
])
def test_aligned_fastpath_knob_selects_the_masked_kernel(gpu, shape, dtype, causal, tiles):
    """TILEDATTN_DISABLE_ALIGNED_FASTPATH=1 makes the launch use the tail-masked kernel on a
    sequence length that is a multiple of both tiles (flash_fwd.py:225-226, 880-921); the
    masked and unmasked kernels agree with each other and with the oracle."""
    import torch

    from tiledattention.kernels import flash_fwd as ff

    q, k, v = inputs(shape, dtype, 60 + shape[2] + shape[3])
    rows = sample_rows(shape[2], 64) if shape[2] >= 2048 else None
    ref = oracle_f32(q, k, v, causal=causal, rows=rows)
    dev = torch.device("cuda:0")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    env = {} if tiles is None else {"tile_m": tiles[0], "tile_n": tiles[1]}
    outs = {}
    for disable in (None, "1"):
        say(f"aligned fast path {dtype} {shape} causal={causal} tiles={tiles} disable={disable}")
        with knobs(disable_aligned_fastpath=disable, **env):
            out = _sdpa(qd, kd, vd, causal=causal)
            plan = next(p for key, p in ff._PLANS.items() if key[0] == qd.shape and key[6] is causal
                        and key[7] == ff._knob_snapshot())
        assert plan.args.aligned == (0 if disable else 1)
        outs[disable] = out
        check_close(as_f32(out, rows), ref, dtype, what=f"disable={disable}")
    diff = float((outs[None].float() - outs["1"].float()).abs().max())
    print(f"[check] masked vs unmasked kernel max_abs_diff={diff:.3e}", flush=True)
    assert diff <= TOL[dtype]
