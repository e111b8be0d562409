"""The call policy in two languages agrees: the Python layer (``flash_fwd._resolve_call``,
the reference-named functions over ``TILEDATTN_*`` knobs) and the library's
``ta_plan_call`` (used by the C++ torch operator and any non-Python caller) resolve the same
tile, accumulation, kernel head dim, padding, aligned fast path, workgroup order, split and
workspace for every shape and knob setting of a grid, on a device of 256 compute units (and
of 304, where the one-wave rules move).  Where one side rejects a request, so does the
other.  On the CPU, no device."""

from __future__ import annotations

import ctypes
import itertools

import pytest

from tiledattention import _lib
from tiledattention.kernels import flash_fwd as ff

KNOB_SETS = [
    {},
    {"TILEDATTN_TILE_M": "64", "TILEDATTN_TILE_N": "64"},
    {"TILEDATTN_TILE_M": "128"},
    {"TILEDATTN_TILE_N": "128"},
    {"TILEDATTN_TILE_M": "128", "TILEDATTN_TILE_N": "128", "TILEDATTN_ACCUM_MODE": "fp16"},
    {"TILEDATTN_ACCUM_MODE": "fp16"},
    {"TILEDATTN_ACCUM_MODE": "FP32"},
    {"TILEDATTN_DISABLE_ALIGNED_FASTPATH": "1"},
    {"TILEDATTN_SCHED": "3"},
    {"TILEDATTN_SCHED": "0", "TILEDATTN_SPLIT": "2"},
    {"TILEDATTN_SPLIT": "pairs"},
    {"TILEDATTN_SPLIT": "off"},
    {"TILEDATTN_SPLIT": "1", "TILEDATTN_TILE_M": "64", "TILEDATTN_TILE_N": "64"},
]
OVERRIDES = [(None, None), ((64, 128), "fp32"), ((128, 64), "fp16"), (None, "fp16")]
SHAPES = [(b, h, s) for b, h in ((1, 1), (1, 8), (2, 16), (4, 16)) for s in (1, 100, 512, 1000, 2048, 4096, 8192, 16384)]
DIMS = (16, 48, 64, 72, 96, 100, 128, 136, 160, 200, 256)


@pytest.fixture(scope="module")
def lib():
    if not _lib.library_path().exists():
        pytest.fail("libtiledattn.so is not built: run __graft_entry__.build() first")
    return _lib.load()


def _python(lib, b, h, s, d, dtype, causal, cu, tile, accum):
    try:
        pol = ff._resolve_call(lib, batch=b, heads=h, seq_len=s, head_dim=d, dtype_code=dtype, causal=causal,
                               compute_units=cu, tile=tile, accum=accum)
    except (ValueError, Exception) as exc:  # noqa: BLE001 - any rejection counts
        return ("error", type(exc).__name__)
    return (pol.tile_m, pol.tile_n, pol.kernel_head_dim, d if pol.pad_in_kernel else 0, pol.accum_code,
            pol.aligned, pol.sched, pol.chunk, 0 if pol.pad_in_kernel else pol.pad_dim, pol.width, pol.ws_bytes)


def _library(lib, b, h, s, d, dtype, causal, cu, tile, accum):
    try:
        knobs = ff._call_knobs(tile, accum)
    except ValueError as exc:
        return ("error", type(exc).__name__)
    out = _lib.CallPlan()
    st = lib.ta_plan_call(b, h, s, d, dtype, int(causal), 0, cu, ctypes.byref(knobs), ctypes.byref(out))
    if st != _lib.TA_OK:
        return ("error", _lib.status_name(lib, st))
    a = out.args
    return (a.tile_m, a.tile_n, a.D, a.d_real, a.accum, a.aligned, a.sched, out.chunk_steps, out.host_pad,
            out.out_width, out.workspace_bytes)


@pytest.mark.parametrize("knobs", KNOB_SETS, ids=lambda k: ",".join(f"{a[10:]}={b}" for a, b in k.items()) or "none")
def test_python_and_library_policies_agree(lib, monkeypatch, knobs):
    for name in ff._KNOBS:
        monkeypatch.delenv(name, raising=False)
    for key, val in knobs.items():
        monkeypatch.setenv(key, val)
    ff._SPLIT_PLANS.clear()
    checked = errors = 0
    for (b, h, s), d, dtype, causal, (tile, accum), cu in itertools.product(
            SHAPES, DIMS, (_lib.TA_FP16, _lib.TA_BF16), (False, True), OVERRIDES, (256, 304)):
        if cu == 304 and (dtype == _lib.TA_FP16 or tile is not None):
            continue
        py = _python(lib, b, h, s, d, dtype, causal, cu, tile, accum)
        cc = _library(lib, b, h, s, d, dtype, causal, cu, tile, accum)
        case = dict(B=b, H=h, S=s, D=d, dtype=dtype, causal=causal, tile=tile, accum=accum, cu=cu)
        if py[0] == "error" or cc[0] == "error":
            assert py[0] == cc[0] == "error", (case, py, cc)
            errors += 1
        else:
            assert py == cc, (case, py, cc)
        checked += 1
    assert checked > 1000
    if not knobs:
        assert errors < checked // 4  # the rejections: head dims and tiles without a kernel


def test_policy_examples(lib):
    """Closed-form examples of the library's plan (the rules in include/tiledattn.h)."""
    def plan(**kw):
        k = _lib.CallKnobs(0, 0, -1, 1, -1, _lib.TA_SPLIT_AUTO)
        for key, val in kw.pop("knobs", {}).items():
            setattr(k, key, val)
        out = _lib.CallPlan()
        args = dict(B=1, H=8, S=8192, D=128, dtype=_lib.TA_BF16, causal=1, cu=256)
        args.update(kw)
        st = lib.ta_plan_call(args["B"], args["H"], args["S"], args["D"], args["dtype"], args["causal"], 0,
                              args["cu"], ctypes.byref(k), ctypes.byref(out))
        assert st == _lib.TA_OK, _lib.last_error(lib)
        return out
    c3 = plan()
    assert (c3.args.tile_m, c3.args.tile_n, c3.args.sched, c3.chunk_steps) == (128, 64, 1, 0)
    assert plan(S=2048).args.tile_m == 64          # 256 blocks of 64 rows fit 256 CUs once
    c4 = plan(B=4, H=16, S=4096, causal=0)
    assert (c4.args.tile_m, c4.args.tile_n) == (128, 128)  # non-causal D = 128, S >= 2048
    pad = plan(D=104)  # a multiple of 8: read in place by the eight-wave kernel
    assert (pad.args.D, pad.args.d_real, pad.host_pad, pad.out_width) == (128, 104, 0, 104)
    pad96 = plan(D=72, S=8192)
    assert (pad96.args.D, pad96.args.d_real) == (96, 72)
    odd = plan(D=99)  # not a multiple of 8: zero-padded on the host
    assert (odd.args.D, odd.args.d_real, odd.host_pad, odd.out_width) == (128, 0, 29, 128)
    split = plan(B=1, H=1, S=16384)
    assert split.chunk_steps != 0 and split.workspace_bytes > 0 and split.args.tile_m == 128
    assert plan(B=1, H=1, S=16384, knobs={"accum": _lib.TA_ACC_INPUT}).chunk_steps == 0
    assert plan(S=8191).args.aligned == 0 and plan(knobs={"aligned": 0}).args.aligned == 0
