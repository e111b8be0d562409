"""ta_sdpa_fwd_split_static, the entry point that allocates nothing, through the C ABI.

It must give exactly what ta_sdpa_fwd_split gives with a caller-owned workspace (the same
kernels; only the workspace's address differs), on two calls in a row whose second is
smaller (the static array keeps the first call's partials), for chunk lengths and the
paired split, and meet the north-star bound against the fp32 oracle.  Torch only allocates the tensors and provides the stream."""

from __future__ import annotations

import ctypes

import pytest

from tests.parity_util import as_f32, check_close, inputs, oracle_f32, say
from tiledattention import _lib

pytestmark = pytest.mark.gpu


def _args(qd, kd, vd, o, *, causal: int, dtype_code: int):
    a = _lib.FwdArgs()
    a.q, a.k, a.v, a.o = qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), o.data_ptr()
    a.B, a.H, a.S, a.D = qd.shape
    for name, t in (("q_stride", qd), ("k_stride", kd), ("v_stride", vd), ("o_stride", o)):
        getattr(a, name)[:] = tuple(t.stride())
    a.scale, a.causal, a.dtype = qd.shape[3] ** -0.5, causal, dtype_code
    a.tile_m, a.tile_n, a.accum, a.device, a.sched, a.aligned = 128, 64, _lib.TA_ACC_FP32, 0, 1, 1
    return a


@pytest.mark.parametrize("order", ["large_then_small", "small_then_large_then_small"])
def test_static_scratch_matches_caller_workspace(gpu, order):
    import torch

    lib = _lib.load()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev).cuda_stream
    big = ((1, 4, 2048, 128), 1, "bfloat16", 3)
    small = ((1, 2, 700, 64), 0, "float16", 1)
    # the paired split (11 blocks a head, 3 pairs cut, the middle block alone)
    pairs = ((1, 3, 1300, 128), 1, "bfloat16", _lib.TA_SPLIT_PAIRS)
    cases = [big, pairs, small] if order == "large_then_small" else [small, big, pairs, small]
    for shape, causal, dtype, chunk in cases:
        dc = _lib.TA_BF16 if dtype == "bfloat16" else _lib.TA_FP16
        q, k, v = inputs(shape, dtype, 90 + shape[2])
        qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
        o_ws = torch.full_like(qd, float("nan"))
        o_st = torch.full_like(qd, float("nan"))
        need = ctypes.c_int64(0)
        a = _args(qd, kd, vd, o_ws, causal=causal, dtype_code=dc)
        assert lib.ta_split_workspace_size(ctypes.byref(a), chunk, ctypes.byref(need)) == _lib.TA_OK
        assert 0 < need.value <= _lib.STATIC_SCRATCH_BYTES
        ws = torch.full((need.value,), 0x7F, dtype=torch.uint8, device=dev)  # garbage workspace
        say(f"static scratch {order}: {dtype} {shape} causal={causal} chunk={chunk} ws={need.value}")
        st = lib.ta_sdpa_fwd_split(ctypes.byref(a), chunk, ctypes.c_void_p(ws.data_ptr()), need.value,
                                   ctypes.c_void_p(stream))
        assert st == _lib.TA_OK, _lib.last_error(lib)
        b = _args(qd, kd, vd, o_st, causal=causal, dtype_code=dc)
        st = lib.ta_sdpa_fwd_split_static(ctypes.byref(b), chunk, ctypes.c_void_p(stream))
        assert st == _lib.TA_OK, _lib.last_error(lib)
        torch.cuda.synchronize()
        # once warm, a call allocates no device memory: the free bytes do not move
        free0 = torch.cuda.mem_get_info(dev)[0]
        st = lib.ta_sdpa_fwd_split_static(ctypes.byref(b), chunk, ctypes.c_void_p(stream))
        assert st == _lib.TA_OK, _lib.last_error(lib)
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info(dev)[0] == free0
        assert torch.equal(o_ws, o_st), float((o_ws.float() - o_st.float()).abs().max())
        check_close(as_f32(o_st), oracle_f32(q, k, v, causal=bool(causal)), dtype,
                    what=f"static scratch {shape}")


def test_static_scratch_whole_rows_and_oversize(gpu):
    """A chunk length that splits nothing runs the whole-row kernel (no scratch); a chunk
    length whose workspace exceeds the static array is rejected before any launch."""
    import torch

    lib = _lib.load()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev).cuda_stream
    q, k, v = inputs((1, 2, 512, 128), "float16", 7)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o0, o1 = torch.empty_like(qd), torch.empty_like(qd)
    say("static scratch: chunk 4 of 4 steps (nothing split) vs ta_sdpa_fwd")
    assert lib.ta_sdpa_fwd(ctypes.byref(_args(qd, kd, vd, o0, causal=1, dtype_code=_lib.TA_FP16)),
                           ctypes.c_void_p(stream)) == _lib.TA_OK
    assert lib.ta_sdpa_fwd_split_static(ctypes.byref(_args(qd, kd, vd, o1, causal=1, dtype_code=_lib.TA_FP16)),
                                        4, ctypes.c_void_p(stream)) == _lib.TA_OK
    torch.cuda.synchronize()
    assert torch.equal(o0, o1)
    check_close(as_f32(o1), oracle_f32(q, k, v, causal=True), "float16", what="static whole rows")
    # B1 H64 S=16384 D=128, chunks of one step: ~4 GiB of partials, far above the array.
    # Null tensor pointers: were the size check ever skipped, validation would still reject
    # the call before any launch.
    a = _args(qd, kd, vd, o1, causal=1, dtype_code=_lib.TA_FP16)
    a.q = a.k = a.v = a.o = None
    a.H, a.S = 64, 16384
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        getattr(a, name)[:] = (64 * 16384 * 128, 16384 * 128, 128, 1)
    say("static scratch: oversize request is rejected")
    assert lib.ta_sdpa_fwd_split_static(ctypes.byref(a), 1, ctypes.c_void_p(stream)) == _lib.TA_EINVAL
    assert "exceeds the static scratch" in _lib.last_error(lib)
