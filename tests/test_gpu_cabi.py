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
