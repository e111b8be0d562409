"""The C ABI driven directly, as a foreign caller would bind it (no Python policy layer):
torch only allocates device memory and provides the stream."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from tests.parity_util import check_close, inputs, oracle_f32, say
from tiledattention import _lib

pytestmark = pytest.mark.gpu


def _fill(a, q, k, v, o, *, causal, dtype_code, tm, tn, accum=0, scale=None):
    b, h, s, d = q.shape
    a.q, a.k, a.v, a.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
    a.B, a.H, a.S, a.D = b, h, s, d
    for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("o_stride", o)):
        getattr(a, name)[:] = tuple(t.stride())
    a.scale = 1.0 / np.sqrt(d) if scale is None else scale
    a.causal, a.dtype, a.tile_m, a.tile_n, a.accum = int(causal), dtype_code, tm, tn, accum
    a.device, a.sched = q.device.index or 0, 0


@pytest.mark.parametrize("tm,tn", [(64, 64), (128, 64), (64, 128), (128, 128)])
def test_cabi_direct_launch_matches_oracle(gpu, tm, tn):
    import torch

    lib = _lib.load()
    q, k, v = inputs((1, 2, 64, 64), "float16", 0)
    ref = oracle_f32(q, k, v, causal=True)
    qd, kd, vd = (t.cuda() for t in (q, k, v))
    od = torch.empty_like(qd)
    a = _lib.FwdArgs()
    _fill(a, qd, kd, vd, od, causal=True, dtype_code=_lib.TA_FP16, tm=tm, tn=tn)
    stream = torch.cuda.Stream()
    say(f"C-ABI ta_sdpa_fwd C1 tiles=({tm},{tn}) on a side stream")
    st = lib.ta_sdpa_fwd(ctypes.byref(a), ctypes.c_void_p(stream.cuda_stream))
    assert st == _lib.TA_OK, _lib.last_error(lib)
    stream.synchronize()
    check_close(od.float().cpu().numpy(), ref, "float16", what=f"C-ABI tiles={tm},{tn}")


def test_cabi_prepare_populates_cache(gpu):
    lib = _lib.load()
    say("C-ABI ta_prepare / ta_cache_reset")
    assert lib.ta_cache_reset() == _lib.TA_OK
    assert lib.ta_cache_size() == 0
    st = lib.ta_prepare(0, _lib.TA_BF16, 128, 128, 64, 1, _lib.TA_ACC_FP32, 1)
    assert st == _lib.TA_OK, _lib.last_error(lib)
    assert lib.ta_cache_size() == 1
    assert lib.ta_prepare(0, _lib.TA_BF16, 128, 128, 64, 1, _lib.TA_ACC_FP32, 1) == _lib.TA_OK
    assert lib.ta_cache_size() == 1
    assert lib.ta_prepare(0, _lib.TA_FP16, 64, 64, 128, 0, _lib.TA_ACC_INPUT, 0) == _lib.TA_OK
    assert lib.ta_cache_size() == 2


def test_cabi_bad_device_is_a_hip_error(gpu):
    import torch

    lib = _lib.load()
    q = torch.zeros((1, 1, 64, 64), dtype=torch.float16, device="cuda")
    a = _lib.FwdArgs()
    _fill(a, q, q, q, q, causal=False, dtype_code=_lib.TA_FP16, tm=64, tn=64)
    a.device = torch.cuda.device_count() + 3
    say("C-ABI invalid device ordinal")
    assert lib.ta_sdpa_fwd(ctypes.byref(a), None) == _lib.TA_EHIP
    assert "device" in _lib.last_error(lib)
    # The failure is reported through the status only: the next torch launch must not
    # find it in the runtime's last-error slot.
    x = torch.ones(4, device="cuda") * 2
    torch.cuda.synchronize()
    assert float(x.sum()) == 8.0


def test_describe_launch_on_the_device(gpu):
    """ta_describe_launch on the device equals the model at the device's CU count, and the
    Python layer's description of a call names the same kernel (the headline workload:
    causal pairs at 256 CUs)."""
    import torch

    from tiledattention.kernels import flash_fwd

    lib = _lib.load()
    cu = torch.cuda.get_device_properties(0).multi_processor_count
    say(f"C-ABI ta_describe_launch on device 0 ({cu} CUs)")
    for kw in (dict(B=1, H=8, S=8192, D=128, causal=True, sched=1),
               dict(B=4, H=16, S=4096, D=128, causal=False, sched=1),
               dict(B=1, H=8, S=512, D=128, causal=True, tile_m=64)):
        args = _lib.shape_args(**kw)
        on_dev = _lib.describe(lib, args).as_dict()
        model = _lib.describe(lib, args, compute_units=cu).as_dict()
        assert on_dev == model and on_dev["compute_units"] == cu
    q, k, v = inputs((1, 8, 8192, 128), "bfloat16", 1234)
    qd, kd, vd = (t.cuda() for t in (q, k, v))
    desc = flash_fwd.describe_call(qd, kd, vd, causal=True)
    expect = "ta_fwd_pp_pair_bf16_d128_c1_t0" if cu <= 256 else "ta_fwd_pp_bf16_d128_c1_t0"
    assert desc["kernel"] == expect and desc["code_object"] == "attn_fwd_pp.hsaco"
