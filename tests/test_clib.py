"""The C-ABI library on the CPU: it loads, exports every function include/tiledattn.h
declares, and rejects bad arguments with the documented status before any HIP call.
No kernel is launched here (there is no GPU in the CPU suite)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from tiledattention import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tiledattn.h"


@pytest.fixture(scope="module")
def lib():
    if not _lib.library_path().exists():
        pytest.fail("libtiledattn.so is not built: run __graft_entry__.build() first")
    return _lib.load()


def _declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:[A-Za-z_][\w\s\*]*?)\b(ta_\w+)\s*\(", text, flags=re.M))


def test_header_and_binding_agree():
    assert _declared_functions() == set(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(str(_lib.library_path()))
    for name in _declared_functions():
        assert hasattr(raw, name), name


def test_abi_version_and_status_names(lib):
    assert lib.ta_abi_version() == _lib.ABI_VERSION == 6
    names = [lib.ta_status_string(i).decode() for i in range(5)]
    assert names == ["TA_OK", "TA_EINVAL", "TA_EUNSUPPORTED", "TA_ENOKERNEL", "TA_EHIP"]
    assert lib.ta_status_string(99).decode() == "TA_UNKNOWN"


def _args(**kw) -> _lib.FwdArgs:
    a = _lib.FwdArgs()
    a.q = a.k = a.v = a.o = 0x10000  # never dereferenced: validation fails or no launch
    a.B, a.H, a.S, a.D = 1, 2, 64, 64
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        getattr(a, name)[:] = (2 * 64 * 64, 64 * 64, 64, 1)
    a.scale, a.causal, a.dtype, a.tile_m, a.tile_n, a.accum, a.device, a.sched = 0.125, 0, 0, 64, 64, 0, 0, 0
    for key, val in kw.items():
        if key.endswith("_stride"):
            getattr(a, key)[:] = val
        else:
            setattr(a, key, val)
    return a


# element strides of dense D = 128 rows (batch and head strides 0: a broadcast slice is valid)
_D128 = {n: (0, 0, 128, 1) for n in ("q_stride", "k_stride", "v_stride", "o_stride")}


def _call(lib, a):
    return lib.ta_sdpa_fwd(ctypes.byref(a), None)


@pytest.mark.parametrize("kw,status,msg", [
    (dict(dtype=2), _lib.TA_EINVAL, "dtype"),
    (dict(accum=5), _lib.TA_EINVAL, "accum"),
    (dict(causal=2), _lib.TA_EINVAL, "causal"),
    (dict(sched=4), _lib.TA_EINVAL, "sched"),
    (dict(S=-1), _lib.TA_EINVAL, "negative"),
    (dict(D=96, accum=1), _lib.TA_EUNSUPPORTED, "head_dim 96 with tile (64, 64)"),
    (dict(D=96, tile_m=128, accum=1), _lib.TA_EUNSUPPORTED, "head_dim 96 with tile (128, 64)"),
    (dict(D=80), _lib.TA_EUNSUPPORTED, "head_dim"),
    (dict(D=160, tile_n=128), _lib.TA_EUNSUPPORTED, "tile_n 128 with head_dim 160"),
    (dict(D=512), _lib.TA_EUNSUPPORTED, "head_dim"),
    (dict(tile_m=32), _lib.TA_EUNSUPPORTED, "tile"),
    (dict(tile_n=256), _lib.TA_EUNSUPPORTED, "tile"),
    (dict(q=0), _lib.TA_EINVAL, "null"),
    (dict(v=0x10008), _lib.TA_EINVAL, "16-byte aligned"),
    (dict(k_stride=(2 * 64 * 64, 64 * 64, 64, 2)), _lib.TA_EINVAL, "last-dim stride"),
    (dict(o_stride=(2 * 64 * 64, 64 * 64, 68, 1)), _lib.TA_EINVAL, "multiple of 8"),
    (dict(S=1 << 24, D=128, **_D128), _lib.TA_EINVAL, "2^31"),
    (dict(S=2, k_stride=(0, 0, 1 << 23, 1)), _lib.TA_EINVAL, "k: row stride 8388608 must stay below 2^23"),
    # a stride large enough that S * stride would overflow int64 is rejected by its bound first
    (dict(S=1 << 30, v_stride=(0, 0, 1 << 60, 1)), _lib.TA_EINVAL, "v: row stride"),
    # Q's range limit applies where Q is staged with buffer loads (the eight-wave kernel)
    (dict(S=1 << 20, D=128, tile_m=128, **{**_D128, "q_stride": (0, 0, 1024, 1)}), _lib.TA_EINVAL,
     "q: S * row stride"),
    (dict(S=2, q_stride=(0, 0, 1 << 23, 1), D=128, tile_m=128), _lib.TA_EINVAL, "q: row stride"),
    # rows that overlap: a zero row stride (k expanded along S) or one below the row width
    (dict(k_stride=(0, 0, 0, 1)), _lib.TA_EINVAL, "k: row stride 0 is below the row width 64"),
    (dict(v_stride=(0, 0, 56, 1)), _lib.TA_EINVAL, "v: row stride 56 is below the row width 64"),
    (dict(D=128, **{**_D128, "o_stride": (0, 0, 120, 1)}), _lib.TA_EINVAL,
     "o: row stride 120"),
    (dict(d_real=96, D=128, tile_m=128, **{**_D128, "k_stride": (0, 0, 88, 1)}), _lib.TA_EINVAL,
     "below the row width 96"),
    (dict(aligned=2), _lib.TA_EINVAL, "aligned 2"),
    (dict(d_real=4), _lib.TA_EINVAL, "d_real 4"),
    (dict(d_real=72), _lib.TA_EINVAL, "d_real 72"),        # above D = 64
    (dict(d_real=-8), _lib.TA_EINVAL, "d_real"),
    (dict(d_real=36, D=128, tile_m=128), _lib.TA_EINVAL, "multiple of 8"),
    (dict(d_real=136, D=160, accum=1, tile_m=128), _lib.TA_EUNSUPPORTED, "d_real needs"),
    (dict(d_real=200, D=256), _lib.TA_EUNSUPPORTED, "d_real needs"),  # 64-row tiles: D <= 160
    (dict(d_real=200, D=256, tile_m=128), _lib.TA_EUNSUPPORTED, "D <= 160"),
])
def test_argument_validation(lib, kw, status, msg):
    st = _call(lib, _args(**kw))
    assert st == status
    assert msg in _lib.last_error(lib)


def test_grid_beyond_32bit_work_items_is_rejected_before_any_device_call(lib):
    """The dispatch packet counts work-items in 32 bits: B1 H1024 S=2^20 D128 on the
    eight-wave kernel is 8192 * 1024 workgroups of 512 threads = 2^32 work-items."""
    s, h, d = 1 << 20, 1024, 128
    st = (h * s * d, s * d, d, 1)
    a = _args(B=1, H=h, S=s, D=d, tile_m=128, tile_n=64, accum=_lib.TA_ACC_FP32,
              q_stride=st, k_stride=st, v_stride=st, o_stride=st)
    assert _call(lib, a) == _lib.TA_EINVAL
    assert "2^32 work-items" in _lib.last_error(lib)


def test_split_grid_beyond_32bit_work_items_is_rejected(lib):
    """Non-causal B1 H512 S=2^20 D128 in 4096-step chunks: 512 heads x 8192 blocks x 2 chunks
    = 2^23 split workgroups of 512 threads = 2^32 work-items."""
    s, h, d = 1 << 20, 512, 128
    st = (h * s * d, s * d, d, 1)
    a = _args(B=1, H=h, S=s, D=d, tile_m=128, tile_n=64, accum=_lib.TA_ACC_FP32,
              q_stride=st, k_stride=st, v_stride=st, o_stride=st)
    need = ctypes.c_int64(0)
    assert lib.ta_split_workspace_size(ctypes.byref(a), 4096, ctypes.byref(need)) == _lib.TA_OK
    assert need.value > 0
    rc = lib.ta_sdpa_fwd_split(ctypes.byref(a), 4096, ctypes.c_void_p(0x100000), need.value, None)
    assert rc == _lib.TA_EINVAL
    assert "split kernel grid" in _lib.last_error(lib)


def test_null_args_pointer(lib):
    assert lib.ta_sdpa_fwd(None, None) == _lib.TA_EINVAL
    assert "NULL" in _lib.last_error(lib)


@pytest.mark.parametrize("kw", [dict(B=0), dict(H=0), dict(S=0)])
def test_zero_size_is_ok_without_launch(lib, kw):
    assert _call(lib, _args(q=0, k=0, v=0, o=0, **kw)) == _lib.TA_OK


@pytest.mark.parametrize("args,status", [
    ((0, 3, 64, 64, 64, 0, 0, 1), _lib.TA_EINVAL),        # dtype
    ((0, 0, 80, 64, 64, 0, 0, 1), _lib.TA_EUNSUPPORTED),  # head dim
    ((0, 0, 96, 64, 64, 0, 1, 1), _lib.TA_EUNSUPPORTED),  # D = 96 with input-dtype accumulation
    ((0, 0, 64, 48, 64, 0, 0, 1), _lib.TA_EUNSUPPORTED),  # tile
    ((0, 0, 64, 64, 64, 0, 9, 1), _lib.TA_EINVAL),        # accum
])
def test_prepare_validation(lib, args, status):
    assert lib.ta_prepare(*args) == status


def test_cache_calls_and_code_object_dir(lib):
    assert lib.ta_cache_reset() == _lib.TA_OK
    assert lib.ta_cache_size() == 0
    assert lib.ta_set_code_object_dir(None) == _lib.TA_EINVAL
    assert lib.ta_set_code_object_dir(str(_lib.lib_dir()).encode()) == _lib.TA_OK


def test_error_text_is_thread_local(lib):
    import threading

    _call(lib, _args(D=80))
    seen = {}

    def other():
        seen["msg"] = _lib.last_error(lib)

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == ""
    assert "head_dim" in _lib.last_error(lib)


def test_code_objects_built_for_gfx950():
    for path in _lib.code_object_paths():
        data = path.read_bytes()
        # hipcc --genco writes a clang offload bundle holding the gfx950 ELF
        assert data.startswith(b"__CLANG_OFFLOAD_BUNDLE__") or data[:4] == b"\x7fELF"
        assert b"amdgcn-amd-amdhsa--gfx950" in data and b"\x7fELF" in data
        names = {"attn_fwd_pp.hsaco": ("ta_fwd_pp_bf16_d128", "ta_fwd_pp_f16_d64"),
                 "attn_fwd_wide.hsaco": ("ta_fwd_wide_bf16_d128", "ta_fwd_wide_f16_d64")}.get(
                     path.name, ("ta_fwd_bf16_d128", "ta_fwd_f16_d64"))
        for name in names:
            assert name.encode() in data


def test_static_scratch_entry_rejects_oversize_before_any_device_call(lib):
    """ta_sdpa_fwd_split_static checks the workspace against its static array first: B1 H64
    S=16384 D=128 causal in one-step chunks needs gigabytes of partials."""
    st = (64 * 16384 * 128, 16384 * 128, 128, 1)
    a = _args(B=1, H=64, S=16384, D=128, tile_m=128, tile_n=64, causal=1,
              q_stride=st, k_stride=st, v_stride=st, o_stride=st)
    need = ctypes.c_int64(0)
    assert lib.ta_split_workspace_size(ctypes.byref(a), 1, ctypes.byref(need)) == _lib.TA_OK
    assert need.value > _lib.STATIC_SCRATCH_BYTES
    assert lib.ta_sdpa_fwd_split_static(ctypes.byref(a), 1, None) == _lib.TA_EINVAL
    assert "exceeds the static scratch of 67108864 bytes" in _lib.last_error(lib)
    assert lib.ta_sdpa_fwd_split_static(None, 1, None) == _lib.TA_EINVAL
    # a chunk that splits something needs the split kernels (none for the D = 256 kernels) ...
    st1000 = (2 * 1000 * 256, 1000 * 256, 256, 1)
    a = _args(D=256, S=1000, q_stride=st1000, k_stride=st1000, v_stride=st1000, o_stride=st1000)
    assert lib.ta_sdpa_fwd_split_static(ctypes.byref(a), 1, None) == _lib.TA_EUNSUPPORTED
    assert "split key ranges need" in _lib.last_error(lib)
    # ... one that splits nothing runs ta_sdpa_fwd on any kernel, whose own checks apply
    # (here the row stride 64 below D = 96), before any device call
    assert lib.ta_sdpa_fwd_split_static(ctypes.byref(_args(D=96)), 1, None) == _lib.TA_EINVAL
    assert "row stride 64 is below the row width 96" in _lib.last_error(lib)
