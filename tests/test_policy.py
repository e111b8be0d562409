"""Knob and dispatch policy, pinned by closed-form case tables.

Every table below is written from the reference source it restates (cited per test), not
from this package's code, so a wrong threshold, a swapped default or a missing strip()
fails here.  These run on the CPU.
"""

from __future__ import annotations

import pytest

from tiledattention._errors import DTypeNotSupportedError, InvalidShapeError
from tiledattention import _lib
from tiledattention.kernels import flash_fwd as ff


# ---------------------------------------------------------------- flash_fwd.py:47-65
@pytest.mark.parametrize("raw,default,expected", [
    (None, 7, 7), ("", 7, 7), ("   ", 7, 7), ("64", None, 64), (" 128 ", None, 128), ("-3", 1, -3),
])
def test_get_env_int(monkeypatch, raw, default, expected):
    if raw is None:
        monkeypatch.delenv("TILEDATTN_X", raising=False)
    else:
        monkeypatch.setenv("TILEDATTN_X", raw)
    assert ff._get_env_int("TILEDATTN_X", default) == expected


def test_get_env_int_rejects_non_integer(monkeypatch):
    monkeypatch.setenv("TILEDATTN_X", "64.0")
    with pytest.raises(ValueError, match="Environment variable TILEDATTN_X must be an integer."):
        ff._get_env_int("TILEDATTN_X", None)


# ---------------------------------------------------------------- flash_fwd.py:68-84
@pytest.mark.parametrize("m,n,expected", [
    ("128", None, (128, 64)),   # unset partner defaults to 64
    (None, "128", (64, 128)),
    ("64", "64", (64, 64)),
    ("128", "128", (128, 128)),
    ("32", None, (32, 64)),     # parsed fine; the gfx950 dispatcher rejects it later
])
def test_resolve_tile_config(monkeypatch, m, n, expected):
    for name, val in (("TILEDATTN_TILE_M", m), ("TILEDATTN_TILE_N", n)):
        if val is None:
            monkeypatch.delenv(name, raising=False)
        else:
            monkeypatch.setenv(name, val)
    assert ff._resolve_tile_config() == expected


@pytest.mark.parametrize("m,n", [("0", "64"), ("64", "-64")])
def test_resolve_tile_config_rejects_non_positive(monkeypatch, m, n):
    monkeypatch.setenv("TILEDATTN_TILE_M", m)
    monkeypatch.setenv("TILEDATTN_TILE_N", n)
    with pytest.raises(ValueError, match="must be positive"):
        ff._resolve_tile_config()


@pytest.mark.parametrize("tm,tn,ok", [(64, 64, True), (64, 128, True), (128, 64, True), (128, 128, True),
                                      (32, 64, False), (64, 256, False), (96, 64, False)])
def test_gfx950_tile_set(tm, tn, ok):
    if ok:
        ff._check_tile_supported(tm, tn)
    else:
        with pytest.raises(ValueError, match="Unsupported tile"):
            ff._check_tile_supported(tm, tn)


# ---------------------------------------------------------------- flash_fwd.py:87-99
def test_kernel_options_defaults_and_parse(monkeypatch):
    assert ff._resolve_kernel_options() == (3, None, None)
    monkeypatch.setenv("TILEDATTN_KERNEL_OPT_LEVEL", "2")
    monkeypatch.setenv("TILEDATTN_KERNEL_OCCUPANCY", "4")
    monkeypatch.setenv("TILEDATTN_KERNEL_NUM_CTAS", "2")
    assert ff._resolve_kernel_options() == (2, 4, 2)
    monkeypatch.setenv("TILEDATTN_KERNEL_OCCUPANCY", "many")
    with pytest.raises(ValueError, match="TILEDATTN_KERNEL_OCCUPANCY must be an integer"):
        ff._resolve_kernel_options()


# ---------------------------------------------------------------- flash_fwd.py:102-146
@pytest.mark.parametrize("raw,expected", [
    (None, "fp32"), ("", "fp32"), ("auto", "fp32"), (" AUTO ", "fp32"),
    ("fp32", "fp32"), (" FP32", "fp32"), ("fp16", "fp16"), ("Fp16 ", "fp16"),
])
def test_resolve_accum_mode(monkeypatch, raw, expected):
    if raw is None:
        monkeypatch.delenv("TILEDATTN_ACCUM_MODE", raising=False)
    else:
        monkeypatch.setenv("TILEDATTN_ACCUM_MODE", raw)
    # a shape where the reference's auto rule (flash_fwd.py:102-120: non-causal, D = 64,
    # S >= 1024) picks the input dtype; on gfx950 auto resolves to fp32 (faster and more
    # accurate here)
    assert ff._resolve_accum_mode(seq_len=2048, head_dim=64, causal=False) == expected


@pytest.mark.parametrize("s,d,causal", [(2048, 64, False), (64, 64, True), (8192, 128, False), (1024, 160, False)])
def test_gfx950_auto_accumulation_is_fp32(s, d, causal):
    assert ff._default_accum_mode_for_shape_gfx950(seq_len=s, head_dim=d, causal=causal) == "fp32"


@pytest.mark.parametrize("raw", ["bf16", "fp8", "32"])
def test_resolve_accum_mode_rejects(monkeypatch, raw):
    monkeypatch.setenv("TILEDATTN_ACCUM_MODE", raw)
    with pytest.raises(ValueError, match="Unsupported TILEDATTN_ACCUM_MODE"):
        ff._resolve_accum_mode(seq_len=64, head_dim=64, causal=False)


# ---------------------------------------------------------------- flash_fwd.py:149-163
@pytest.mark.parametrize("d,expected", [
    (1, (64, 63)), (32, (64, 32)), (64, (64, 0)), (65, (128, 63)), (96, (128, 32)), (128, (128, 0)),
    (129, (160, 31)), (160, (160, 0)), (161, (256, 95)), (192, (256, 64)), (256, (256, 0)),
])
def test_gfx950_head_dim_padding(d, expected):
    assert ff._resolve_kernel_head_dim_gfx950(d) == expected


@pytest.mark.parametrize("d,expected", [
    (64, (64, 0)), (65, (96, 31)), (72, (96, 24)), (96, (96, 0)), (97, (128, 31)), (128, (128, 0)),
    (160, (160, 0)),
])
def test_gfx950_native_96_head_dim(d, expected):
    """128-row tiles with fp32 accumulation have a D = 96 kernel: head dims in (64, 96] run
    on it (padding to 96, not 128); the other paths keep the D = 128 kernel."""
    assert ff._resolve_kernel_head_dim_gfx950(d, native_96=True) == expected
    if 64 < d <= 96:
        assert ff._resolve_kernel_head_dim_gfx950(d) == (128, 128 - d)
        desc = _lib.describe(_lib.load(), _lib.shape_args(S=512, D=96, causal=True), 0, compute_units=256)
        assert (desc.code_object, desc.kernel) == (b"attn_fwd_pp.hsaco", b"ta_fwd_pp_bf16_d96_c1_t0")


@pytest.mark.parametrize("d", [0, -1, 257, 512])
def test_gfx950_head_dim_rejects(d):
    with pytest.raises(InvalidShapeError):
        ff._resolve_kernel_head_dim_gfx950(d)


# ---------------------------------------------------------------- flash_fwd.py:166-196
@pytest.mark.parametrize("raw,d,expected", [
    (None, 96, None), ("", 96, None), ("96", 96, ((0, 64), (64, 32))),
    ("160", 160, ((0, 128), (128, 32))), ("96,160", 160, ((0, 128), (128, 32))),
    (" 96 , 160 ", 96, ((0, 64), (64, 32))), ("96", 128, None), ("64", 64, None), ("96,", 96, ((0, 64), (64, 32))),
])
def test_resolve_chunk_plan(monkeypatch, raw, d, expected):
    if raw is None:
        monkeypatch.delenv("TILEDATTN_CHUNKED_HEAD_DIMS", raising=False)
    else:
        monkeypatch.setenv("TILEDATTN_CHUNKED_HEAD_DIMS", raw)
    assert ff._resolve_chunk_plan(d) == expected


def test_resolve_chunk_plan_rejects(monkeypatch):
    monkeypatch.setenv("TILEDATTN_CHUNKED_HEAD_DIMS", "96,x")
    with pytest.raises(ValueError, match="comma-separated list of integers"):
        ff._resolve_chunk_plan(96)


# ---------------------------------------------------------------- flash_fwd.py:199-238
@pytest.mark.parametrize("s,tm,tn,expected", [
    (1024, 64, 64, True), (1024, 128, 64, True), (1024, 128, 128, True), (1088, 64, 128, False),
    (1152, 128, 64, True), (100, 64, 64, False), (64, 128, 64, False), (8192, 128, 64, True),
])
def test_unmasked_tail_kernel_predicate(s, tm, tn, expected):
    assert ff._use_unmasked_tail_kernel(seq_len=s, tile_m=tm, tile_n=tn) is expected


@pytest.mark.parametrize("raw,expected", [("", True), ("0", True), ("false", True), ("False", True),
                                          (" 0 ", True), ("1", False), ("true", False),
                                          ("FALSE", False), ("yes", False)])
def test_aligned_fastpath_disable_env(monkeypatch, raw, expected):
    # the reference's parse (flash_fwd.py:225-226): only "", "0", "false", "False" keep it on
    monkeypatch.setenv("TILEDATTN_DISABLE_ALIGNED_FASTPATH", raw)
    assert ff._use_unmasked_tail_kernel(seq_len=1024, tile_m=64, tile_n=64) is expected


_D = 128


@pytest.mark.parametrize("shape,stride,width,ok", [
    ((1, 2, 64, _D), (2 * 64 * _D, 64 * _D, _D, 1), _D, True),      # dense
    ((1, 2, 64, _D), (64 * 4 * _D, _D, 4 * _D, 1), _D, True),       # [B,S,H,D] transposed
    ((1, 2, 64, _D), (0, 0, _D, 1), _D, True),                      # broadcast (b, h)
    ((1, 2, 64, _D), (0, 64 * _D, 0, 1), _D, False),                # expanded along S
    ((1, 2, 1, _D), (0, _D, 0, 1), _D, False),                      # S = 1, zero row stride
    ((1, 2, 64, _D), (0, 0, 120, 1), _D, False),                    # overlapping rows
    ((1, 2, 64, 96), (0, 0, 96, 1), 96, True),                      # in-kernel padded width
    ((1, 2, 64, 96), (0, 0, 96, 1), _D, False),                     # needs a host pad
    ((1, 2, 64, _D), (0, 0, 132, 1), _D, False),                    # 16-byte rows
    ((1, 2, 64, _D), (0, 0, _D, 2), _D, False),                     # last stride
    ((1, 1, 2, _D), (0, 0, 1 << 23, 1), _D, False),                 # 128 rows >= 2^31 bytes
    ((1, 1, (1 << 16) - 1, _D), (0, 0, 1 << 14, 1), _D, True),      # slice = 2^31 - 2^15 bytes
    ((1, 1, 1 << 16, _D), (0, 0, 1 << 14, 1), _D, False),           # slice = 2^31 bytes
])
def test_strides_kernel_ready(shape, stride, width, ok):
    """Which views the kernels read in place; the rest are copied to dense tensors (the C ABI
    rejects them with TA_EINVAL, tests/test_clib.py)."""
    assert ff._strides_ok(stride, shape, width) is ok



# ---------------------------------------------------------------- flash_fwd.py:805-818
@pytest.mark.parametrize("raw,expected", [(None, "async"), ("post", "post"), (" STRICT ", "strict"),
                                          ("Async", "async")])
def test_sync_mode(monkeypatch, raw, expected):
    if raw is None:
        monkeypatch.delenv("TILEDATTN_SYNC_MODE", raising=False)
    else:
        monkeypatch.setenv("TILEDATTN_SYNC_MODE", raw)
    assert ff._resolve_sync_mode() == expected


def test_sync_mode_rejected_before_launch(monkeypatch):
    monkeypatch.setenv("TILEDATTN_SYNC_MODE", "eventually")
    with pytest.raises(ValueError, match="Unsupported TILEDATTN_SYNC_MODE='eventually'"):
        ff._resolve_sync_mode()


# ---------------------------------------------------------------- flash_fwd.py:27-44
def test_dtype_codes():
    import torch

    assert ff._dtype_code_for_torch_dtype(torch.float16) == 0
    assert ff._dtype_code_for_torch_dtype(torch.bfloat16) == 1
    with pytest.raises(DTypeNotSupportedError, match="float16 or torch.bfloat16"):
        ff._dtype_code_for_torch_dtype(torch.float32)


# ---------------------------------------------------------------- workgroup order (this build)
@pytest.mark.parametrize("n,causal,tiles,accum,d,expected", [
    (512, True, (128, 64), "fp32", 128, 1),   # C3 S=8192: eight-wave kernel, one per CU -> heavy first
    (256, True, (128, 64), "fp32", 128, 2),   # every workgroup resident
    (512, True, (128, 64), "fp32", 64, 1),    # causal eight-wave D=64: one per CU, heavy first
    (256, True, (128, 64), "fp32", 64, 2),
    (512, True, (128, 64), "input", 128, 1),  # eight-wave input-dtype kernel: one per CU
    (256, True, (128, 64), "input", 128, 2),
    (512, True, (128, 64), "input", 160, 2),  # four-wave kernel (D = 160): all 512 resident (2 per CU)
    (1024, True, (128, 64), "input", 160, 1),
    (256, True, (128, 128), "fp32", 128, 2),
    (512, True, (128, 128), "fp32", 128, 1),
    (512, True, (128, 128), "fp32", 64, 1),   # other tiles: one per CU at any D
    (512, False, (128, 64), "fp32", 64, 1),
    (12, True, (128, 64), "fp32", 128, 0),    # does not split over the 8 XCDs
])
def test_sched_default(n, causal, tiles, accum, d, expected):
    if not causal:
        assert ff._workgroups_per_cu(tile_m=tiles[0], tile_n=tiles[1], accum_code=_lib.TA_ACC_FP32,
                                     head_dim=d, causal=False) == (2 if tiles == (128, 64) and d <= 64 else 1)
    code = _lib.TA_ACC_FP32 if accum == "fp32" else _lib.TA_ACC_INPUT
    assert ff._resolve_sched(n_blocks=n, causal=causal, tile_m=tiles[0], tile_n=tiles[1],
                             accum_code=code, head_dim=d, compute_units=256) == expected


def test_sched_env(monkeypatch):
    monkeypatch.setenv("TILEDATTN_SCHED", "0")
    assert ff._resolve_sched(n_blocks=512, causal=True, tile_m=128, tile_n=64, compute_units=256) == 0
    monkeypatch.setenv("TILEDATTN_SCHED", "3")
    assert ff._resolve_sched(n_blocks=512, causal=True, tile_m=128, tile_n=64, compute_units=256) == 3
    for bad in ("4", "-1", "x"):
        monkeypatch.setenv("TILEDATTN_SCHED", bad)
        with pytest.raises(ValueError, match="TILEDATTN_SCHED"):
            ff._resolve_sched(n_blocks=512, causal=True, tile_m=128, tile_n=64, compute_units=256)


# ---------------------------------------------------------------- default tile on gfx950

@pytest.mark.parametrize("s,d,n_bh,accum,expected", [
    (8192, 128, 8, "fp32", (128, 64)),   # C3: 1024 blocks of 64 rows > 256 CUs
    (2048, 128, 8, "fp32", (64, 64)),    # 256 blocks of 64 rows fit the CUs once
    (1024, 128, 8, "fp32", (64, 64)),
    (2049, 128, 8, "fp32", (128, 64)),   # 8 * 33 > 256
    (1024, 128, 32, "fp32", (128, 64)),  # B2 H16: 512 blocks of 64 rows
    (512, 64, 8, "fp32", (64, 64)),
    (512, 96, 8, "fp32", (64, 64)),      # kernel head dim 128 (in-place padding)
    (512, 160, 8, "fp32", (64, 64)),     # the 64-row eight-wave kernel at D = 160
    (2048, 144, 8, "fp32", (64, 64)),    # kernel head dim 160 (in-place padding)
    (4096, 160, 8, "fp32", (128, 64)),   # 512 blocks of 64 rows
    (512, 200, 8, "fp32", (128, 64)),    # kernel head dim 256: the four-wave kernel
    (512, 128, 8, "fp16", (64, 64)),     # input-dtype accumulation: its 64-row eight-wave kernel
    (512, 160, 8, "fp16", (128, 64)),    # D = 160: the four-wave kernels
    (512, 128, 0, "fp32", (128, 64)),    # no head count given
])
def test_default_tile_prefers_64_rows_when_one_wave_of_blocks_fits(s, d, n_bh, accum, expected):
    assert ff._default_tile_config_for_shape_gfx950(seq_len=s, head_dim=d, causal=True, n_bh=n_bh,
                                                    accum_mode=accum, compute_units=256) == expected


@pytest.mark.parametrize("s,d,causal,n_bh,expected", [
    (4096, 128, False, 64, (128, 128)),  # C4 D = 128: the reference's wider key tile
    (2048, 128, False, 64, (128, 128)),
    (2048, 128, False, 8, (64, 128)),    # 64-row blocks fit the CUs once
    (2047, 128, False, 64, (128, 64)),   # S below 2048
    (4096, 128, True, 64, (128, 64)),    # causal
    (4096, 64, False, 64, (128, 64)),    # D = 64 (C4 D = 64)
    (4096, 96, False, 64, (128, 64)),    # the caller's head dim, not the kernel's
])
def test_default_tile_n_follows_the_reference_rule(s, d, causal, n_bh, expected):
    """TILE_N = 128 for non-causal D = 128 at S >= 2048, else 64 (flash_fwd.py:254-259): the
    rounding cadence of input-dtype accumulation matches the reference's default."""
    for accum in ("fp32", "fp16"):
        assert ff._default_tile_config_for_shape_gfx950(seq_len=s, head_dim=d, causal=causal, n_bh=n_bh,
                                                        accum_mode=accum, compute_units=256) == expected




# ---------------------------------------------------------------- split preference and accumulation
def test_split_preference_needs_fp32_accumulation(monkeypatch):
    """Split kernels exist for fp32 accumulation only: a long, narrow causal grid that the
    fp32 planner splits (B1 H1 S16384 D128) keeps the 64-row default under input-dtype
    accumulation instead of moving to 128 rows it could not split."""
    lib = _lib.load()
    assert lib.ta_split_plan_model(16384, 1, 1, 256) != 0
    monkeypatch.delenv("TILEDATTN_SPLIT", raising=False)
    assert ff._split_preferred(lib, 1, 1, 16384, 128, True, 256, "fp16") is False
    monkeypatch.setenv("TILEDATTN_SPLIT", "4")  # forced: fp32 prefers the split tile
    assert ff._split_preferred(lib, 1, 1, 16384, 128, True, 256, "fp32") is True
    assert ff._split_preferred(lib, 1, 1, 16384, 128, True, 256, "fp16") is False
