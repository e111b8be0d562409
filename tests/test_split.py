"""Split key ranges on the CPU: the grid numbering the kernels and the host share
(tiledattention_amd/csrc/attn_fwd_split.h, checked by a host-only C++ program), the
library's dispatch model and workspace sizes through the C ABI, and the
``TILEDATTN_SPLIT`` knob.  No kernel is launched here."""

from __future__ import annotations

import ctypes
import math
import shutil
import subprocess
from pathlib import Path

import pytest

from tiledattention import _lib
from tiledattention.kernels import flash_fwd

ROOT = Path(__file__).resolve().parents[1]
MI355X_CUS = 256


@pytest.fixture(scope="module")
def lib():
    if not _lib.library_path().exists():
        pytest.fail("libtiledattn.so is not built: run __graft_entry__.build() first")
    return _lib.load()


def test_grid_numbering_covers_every_key_step_once(tmp_path):
    """Whole-row and split grids over 1888 (S, B*H, causal, chunk, order) cases: every key
    step of every (b, h, query block) is computed by exactly one workgroup, partial slots
    are unique and in range, and the merge grid names exactly the split blocks with their
    chunks' slots in key order."""
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "split_numbering_check"
    subprocess.run(
        [gxx, "-O1", "-std=c++17", "-Wall", "-Werror", f"-I{ROOT / 'tiledattention_amd' / 'csrc'}",
         "-o", str(exe), str(ROOT / "tests" / "native" / "split_numbering_check.cpp")],
        check=True, capture_output=True, text=True,
    )
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout[-2000:]
    assert res.stdout.startswith("ok ")


def _args(*, S, B=1, H=8, D=128, causal=1, tile_m=128, tile_n=64, accum=_lib.TA_ACC_FP32, dtype=_lib.TA_BF16):
    a = _lib.FwdArgs()
    a.B, a.H, a.S, a.D = B, H, S, D
    a.scale, a.causal, a.dtype = 0.125, causal, dtype
    a.tile_m, a.tile_n, a.accum, a.device, a.sched = tile_m, tile_n, accum, 0, 1
    return a


def _slots(S: int, causal: bool, chunk: int) -> int:
    """Chunks of the query blocks that have more than one chunk, per (b, h)."""
    steps_total = math.ceil(S / 128)
    total = 0
    for qt in range(math.ceil(S / 128)):
        steps = min(qt + 1, steps_total) if causal else steps_total
        ns = math.ceil(steps / chunk)
        if ns > 1:
            total += ns
    return total


@pytest.mark.parametrize("S", [129, 1000, 1024, 2048, 4096, 5000])
@pytest.mark.parametrize("causal", [0, 1])
@pytest.mark.parametrize("chunk", [1, 2, 3, 7, 16])
@pytest.mark.parametrize("D", [64, 128, 160])
def test_workspace_size_is_one_fp32_partial_per_chunk_of_a_split_block(lib, S, causal, chunk, D):
    a = _args(S=S, B=2, H=3, D=D, causal=causal)
    out = ctypes.c_int64(-1)
    assert lib.ta_split_workspace_size(ctypes.byref(a), chunk, ctypes.byref(out)) == _lib.TA_OK
    rows = 6 * _slots(S, bool(causal), chunk) * 128
    expect = (rows * D * 4 + 255) // 256 * 256 + rows * 4 if rows else 0
    assert out.value == expect


def test_workspace_size_edge_cases(lib):
    out = ctypes.c_int64(-1)
    assert lib.ta_split_workspace_size(ctypes.byref(_args(S=4096)), 0, ctypes.byref(out)) == _lib.TA_OK
    assert out.value == 0
    assert lib.ta_split_workspace_size(ctypes.byref(_args(S=4096)), -2, ctypes.byref(out)) == _lib.TA_EINVAL
    # a chunk as long as the longest row splits nothing
    assert lib.ta_split_workspace_size(ctypes.byref(_args(S=4096)), 32, ctypes.byref(out)) == _lib.TA_OK
    assert out.value == 0
    for kw in (dict(accum=_lib.TA_ACC_INPUT), dict(tile_m=64, accum=_lib.TA_ACC_INPUT),
               dict(tile_n=128, accum=_lib.TA_ACC_INPUT), dict(D=256)):
        st = lib.ta_split_workspace_size(ctypes.byref(_args(S=4096, **kw)), 4, ctypes.byref(out))
        assert st == _lib.TA_EUNSUPPORTED, kw
        assert "split key ranges" in _lib.last_error(lib)
    # 64-row tiles split chunks (the 128-row numbering and workspace), not the paired split
    ref = ctypes.c_int64(0)
    assert lib.ta_split_workspace_size(ctypes.byref(_args(S=4096)), 4, ctypes.byref(ref)) == _lib.TA_OK
    for kw in (dict(tile_m=64), dict(tile_m=64, tile_n=128)):
        assert lib.ta_split_workspace_size(ctypes.byref(_args(S=4096, **kw)), 4, ctypes.byref(out)) == _lib.TA_OK
        assert out.value == ref.value > 0
        st = lib.ta_split_workspace_size(ctypes.byref(_args(S=4096, causal=1, **kw)), _lib.TA_SPLIT_PAIRS,
                                         ctypes.byref(out))
        assert st == _lib.TA_EUNSUPPORTED and "paired split" in _lib.last_error(lib)
    assert lib.ta_split_workspace_size(None, 4, ctypes.byref(out)) == _lib.TA_EINVAL


def test_split_launch_rejects_bad_workspace_before_any_device_call(lib):
    a = _args(S=4096)
    a.q = a.k = a.v = a.o = 0x10000
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        getattr(a, name)[:] = (8 * 4096 * 128, 4096 * 128, 128, 1)
    need = ctypes.c_int64(0)
    assert lib.ta_split_workspace_size(ctypes.byref(a), 4, ctypes.byref(need)) == _lib.TA_OK
    assert need.value > 0
    st = lib.ta_sdpa_fwd_split(ctypes.byref(a), 4, ctypes.c_void_p(0x100000), need.value - 4, None)
    assert st == _lib.TA_EINVAL and "workspace of" in _lib.last_error(lib)
    st = lib.ta_sdpa_fwd_split(ctypes.byref(a), 4, None, need.value, None)
    assert st == _lib.TA_EINVAL and "workspace of" in _lib.last_error(lib)
    st = lib.ta_sdpa_fwd_split(ctypes.byref(a), 4, ctypes.c_void_p(0x100010), need.value, None)
    assert st == _lib.TA_EINVAL and "256-byte" in _lib.last_error(lib)
    st = lib.ta_sdpa_fwd_split(ctypes.byref(a), -2, ctypes.c_void_p(0x100000), need.value, None)
    assert st == _lib.TA_EINVAL
    a.accum = _lib.TA_ACC_INPUT  # no split kernels with input-dtype accumulation
    st = lib.ta_sdpa_fwd_split(ctypes.byref(a), 4, ctypes.c_void_p(0x100000), need.value, None)
    assert st == _lib.TA_EUNSUPPORTED


def _cut_pairs(nq: int, f: int = 4) -> int:
    """Pairs the paired split cuts: p with (nq - 2p - 1 - f) // 2 > 0 (the library's cut
    offset f is 4 key steps)."""
    return sum(1 for p in range(nq // 2) if (nq - 2 * p - 1 - f) // 2 > 0)


@pytest.mark.parametrize("S,D", [(4096, 128), (1000, 64), (1300, 160), (2100, 96), (8192, 128),
                                 (129, 128), (900, 128)])
def test_paired_split_workspace_is_two_partials_per_cut_pair(lib, S, D):
    a = _args(S=S, B=2, H=3, D=D, causal=1)
    out = ctypes.c_int64(-1)
    assert lib.ta_split_workspace_size(ctypes.byref(a), _lib.TA_SPLIT_PAIRS, ctypes.byref(out)) == _lib.TA_OK
    rows = 6 * 2 * _cut_pairs(math.ceil(S / 128)) * 128
    assert out.value == ((rows * D * 4 + 255) // 256 * 256 + rows * 4 if rows else 0)
    # S = 4096: 32 blocks, pairs p = 0 .. 12 cut (k_p = 13 .. 1 steps)
    if S == 4096:
        assert rows == 6 * 2 * 13 * 128
    # non-causal: the paired split is the whole-row grid (no workspace)
    a.causal = 0
    assert lib.ta_split_workspace_size(ctypes.byref(a), _lib.TA_SPLIT_PAIRS, ctypes.byref(out)) == _lib.TA_OK
    assert out.value == 0


def test_split_knob_pairs(monkeypatch, lib):
    a = _args(S=4096)
    monkeypatch.setenv("TILEDATTN_SPLIT", "pairs")
    assert flash_fwd._resolve_split(lib, a, capable=True) == _lib.TA_SPLIT_PAIRS
    with pytest.raises(ValueError, match="TILEDATTN_SPLIT needs"):
        flash_fwd._resolve_split(lib, a, capable=False)
    monkeypatch.setenv("TILEDATTN_SPLIT", "pair")
    with pytest.raises(ValueError, match="'pairs'"):
        flash_fwd._resolve_split(lib, a, capable=True)
    desc = _lib.describe(lib, _lib.shape_args(S=4096, H=8, causal=True), _lib.TA_SPLIT_PAIRS,
                         compute_units=MI355X_CUS)
    assert (desc.code_object, desc.kernel) == (b"attn_fwd_pp.hsaco", b"ta_fwd_pp_psplit_bf16_d128_c1_t0")


def _plan(lib, S, n_bh, causal, cus=MI355X_CUS):
    return lib.ta_split_plan_model(S, n_bh, causal, cus)


def test_plan_model_splits_small_grids_and_leaves_large_ones(lib):
    # Measured on the MI355X (B*H, S): splitting made B*H = 1 or 2 with long rows 1.3-2.5x
    # faster (e.g. causal (1, 8192): 84 -> 34 us), while for B*H = 8 (the C3 sweep) the best
    # chunk gained at most 10 % and most chunks lost; the model picks only the former.
    for n_bh, S, causal in ((1, 8192, 1), (1, 16384, 1), (2, 4096, 1), (2, 8192, 1),
                            (2, 4096, 0), (1, 8192, 0)):
        c = _plan(lib, S, n_bh, causal)
        assert 0 < c < S // 128, (n_bh, S, causal, c)
        out = ctypes.c_int64(0)
        a = _args(S=S, B=1, H=n_bh, causal=causal)
        assert lib.ta_split_workspace_size(ctypes.byref(a), c, ctypes.byref(out)) == _lib.TA_OK
        assert out.value > 0  # the chosen chunk splits something
    for S in (1024, 2048, 8192, 16384):
        assert _plan(lib, S, 8, 1) == 0, S
    # causal grids of more than half and at most one 128-row block per CU, 32 blocks a head
    # or more: the paired split (B1 H8 S4096 45.0 -> 44.0 us, fp16 D = 64 33.0 -> 30.2; B1
    # H4 S8192 70.8 with the best chunk, 70.6 paired)
    for S, n_bh in ((4096, 8), (8192, 4), (4096, 6), (8000, 4), (16384, 2)):
        assert _plan(lib, S, n_bh, 1) == _lib.TA_SPLIT_PAIRS, (S, n_bh)
    # shorter rows: the whole-row grid (B1 H16 S2048 24.5 us, 28.5 paired)
    assert _plan(lib, 2048, 16, 1) == 0
    for S, n_bh in ((4096, 8), (8192, 4)):
        assert _plan(lib, S, n_bh, 0) == 0, (S, n_bh)  # non-causal rows are all equal
    # half a wave or less: chunks (B1 H2 S8192 47.2 us against 51.0 paired)
    assert _plan(lib, 8192, 2, 1) > 0 and _plan(lib, 4096, 4, 1) != _lib.TA_SPLIT_PAIRS
    # grids of many waves balance by themselves
    assert _plan(lib, 4096, 64, 1) == 0
    assert _plan(lib, 4096, 64, 0) == 0
    assert _plan(lib, 8192, 32, 0) == 0
    # nothing to split: a single key step
    assert _plan(lib, 128, 1, 1) == 0 and _plan(lib, 100, 1, 0) == 0
    # invalid sizes
    assert _plan(lib, 0, 8, 1) == 0 and _plan(lib, 4096, 0, 1) == 0 and _plan(lib, 4096, 8, 1, 0) == 0


def test_plan_model_uses_the_compute_unit_count(lib):
    # On a device an eighth the size the same grid is several waves deep: no split.
    assert _plan(lib, 8192, 1, 1, MI355X_CUS) > 0
    assert _plan(lib, 8192, 1, 1, 32) == 0


def _plan64(lib, S, n_bh, causal, d=128, cus=MI355X_CUS):
    return lib.ta_split_plan_model_rows(S, n_bh, causal, d, 64, cus)


def _split_items(S, causal, c):
    """Items of the split grid: causal 128-row block i holds i + 1 key steps of 128 keys,
    cut into ceil((i + 1) / c) chunks; non-causal blocks all hold ceil(S / 128) steps."""
    nq = -(-S // 128)
    if causal:
        return sum(-(-(i + 1) // c) for i in range(nq))
    return nq * -(-nq // c)


def test_plan_model_rows64_matches_measured_picks(lib):
    # MI355X timings (us, bf16): whole 64-row blocks against the chosen chunk length.
    # D128 causal B*H 1 S2048 17.2 -> 14.1 (chunks of 4), S4096 28.7 -> 17.6; D64 causal
    # B*H 1 S4096 21.0 -> 14.8; D160 non-causal B*H 2 S4096 33.4 -> 32.5.
    for S, n_bh, causal, d in ((2048, 1, 1, 128), (4096, 1, 1, 128), (4096, 1, 1, 64),
                               (4096, 2, 0, 160), (2048, 2, 1, 128), (8192, 1, 0, 96)):
        c = _plan64(lib, S, n_bh, causal, d)
        assert c > 0, (S, n_bh, causal, d)
        # every workgroup resident at once: two 64-row halves per item, one per CU
        assert 2 * n_bh * _split_items(S, causal, c) <= MI355X_CUS, (S, n_bh, causal, d, c)
    # whole rows where they were as fast or faster: a full chip of 64-row blocks (D128
    # non-causal B*H 4 S2048 17.7 whole against 20.4 split; D160 20.0 against 23.1), short
    # rows (S1024: one workgroup's fixed cost dominates), D96 B*H 2 S2048 (14.3 against 14.9)
    for S, n_bh, causal, d in ((2048, 4, 0, 128), (2048, 4, 0, 160), (1024, 1, 1, 128),
                               (1024, 2, 0, 64), (2048, 2, 0, 96), (2048, 4, 1, 96)):
        assert _plan64(lib, S, n_bh, causal, d) == 0, (S, n_bh, causal, d)
    # outside the region the planner covers (64-row blocks fill more than half the CUs)
    assert _plan64(lib, 8192, 2, 1) == 0 and _plan64(lib, 4096, 8, 0) == 0
    assert _plan64(lib, 8192, 1, 1, cus=128) == 0
    # other row counts: 128 is the 128-row model, anything else no plan
    for S, n_bh, causal in ((8192, 1, 1), (4096, 8, 1), (2048, 16, 1)):
        assert lib.ta_split_plan_model_rows(S, n_bh, causal, 128, 128, MI355X_CUS) == \
            _plan(lib, S, n_bh, causal)
    assert lib.ta_split_plan_model_rows(4096, 1, 1, 128, 256, MI355X_CUS) == 0
    assert _plan64(lib, 0, 1, 1) == 0 and _plan64(lib, 4096, 0, 1) == 0
    assert _plan64(lib, 4096, 1, 1, cus=0) == 0


# ---------------------------------------------------------------- TILEDATTN_SPLIT knob

@pytest.mark.parametrize("raw,capable,expect", [
    ("off", True, 0), ("0", True, 0), ("OFF", False, 0), ("auto", False, 0), ("", False, 0),
    ("3", True, 3), (" 12 ", True, 12), ("0", False, 0),
])
def test_split_knob(monkeypatch, raw, capable, expect):
    monkeypatch.setenv("TILEDATTN_SPLIT", raw)
    assert flash_fwd._resolve_split(None, _args(S=4096), capable=capable) == expect


@pytest.mark.parametrize("raw,capable,msg", [
    ("-1", True, ">= 0"), ("x", True, "'auto', 'off', 'pairs' or an integer"), ("1.5", True, "integer"),
    ("4", False, "tile (128, 64)"),
])
def test_split_knob_rejects(monkeypatch, raw, capable, msg):
    monkeypatch.setenv("TILEDATTN_SPLIT", raw)
    with pytest.raises(ValueError, match=msg.replace("(", r"\(").replace(")", r"\)")):
        flash_fwd._resolve_split(None, _args(S=4096), capable=capable)


def test_split_capability_rule():
    ok = dict(tile_m=128, tile_n=64, accum_code=_lib.TA_ACC_FP32, kernel_head_dim=128)
    rule = flash_fwd._split_capable
    assert rule(**ok)
    assert rule(**{**ok, "kernel_head_dim": 64})
    assert rule(**{**ok, "kernel_head_dim": 160})
    assert not rule(**{**ok, "kernel_head_dim": 256})
    assert rule(**{**ok, "tile_m": 64})  # the 64-row eight-wave kernel splits chunks too
    assert not rule(**{**ok, "tile_m": 64, "accum_code": _lib.TA_ACC_INPUT})
    assert rule(**{**ok, "tile_n": 128})  # the eight-wave step is 128 keys
    assert not rule(**{**ok, "accum_code": _lib.TA_ACC_INPUT})
    # in-place padding (d_real) exists on both eight-wave forms
    ew = flash_fwd._eight_wave_kernel
    assert ew(**ok) and ew(**{**ok, "tile_m": 64}) and ew(**{**ok, "tile_m": 64, "tile_n": 128})
    assert ew(**{**ok, "tile_m": 64, "kernel_head_dim": 160})
    assert not ew(**{**ok, "tile_m": 64, "kernel_head_dim": 256})


# ---------------------------------------------------------------- launch-plan cache keys

def test_knob_snapshot_follows_the_environment(monkeypatch):
    """Launch plans are cached per knob values, so the snapshot must see every change made
    through os.environ (the reference re-reads its knobs on every call)."""
    for name in flash_fwd._KNOBS:
        monkeypatch.delenv(name, raising=False)
    base = flash_fwd._knob_snapshot()
    assert base == (None,) * len(flash_fwd._KNOBS)
    for i, name in enumerate(flash_fwd._KNOBS):
        monkeypatch.setenv(name, "7")
        snap = flash_fwd._knob_snapshot()
        assert snap[i] is not None and snap != base, name
        monkeypatch.delenv(name)
        assert flash_fwd._knob_snapshot() == base
    # every TILEDATTN_* knob the host path reads is part of the key
    src = (ROOT / "tiledattention" / "kernels" / "flash_fwd.py").read_text()
    import re

    read = set(re.findall(r'"(TILEDATTN_[A-Z_]+)"', src))
    assert read == set(flash_fwd._KNOBS)


def test_plan_model_paired_split_boundaries(lib):
    """The paired split's rule: causal, more than CUs / 2 and at most CUs query blocks of 128
    rows, 32 or more a head; the edges of each condition, on 256 and 304 CUs."""
    P = _lib.TA_SPLIT_PAIRS
    assert _plan(lib, 4096, 8, 1) == P            # 256 blocks = CUs
    assert _plan(lib, 4096, 5, 1) == P            # 160 > 128
    assert _plan(lib, 4096, 4, 1) != P            # 128: not more than half
    assert _plan(lib, 4096, 9, 1) != P            # 288 > 256
    assert _plan(lib, 3968, 8, 1) != P            # 31 blocks a head
    assert _plan(lib, 3969, 8, 1) == P            # 32 blocks (ragged last one)
    assert _plan(lib, 4096, 9, 1, cus=304) == P   # 288 <= 304
    assert _plan(lib, 4096, 4, 1, cus=304) != P   # 128 <= 152
    assert _plan(lib, 8192, 3, 0) != P            # non-causal
