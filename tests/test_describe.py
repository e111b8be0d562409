"""The library's own description of a launch (``ta_describe_launch_model``), on the CPU.

Every expectation below is written from the dispatch rules as the header states them
(include/tiledattn.h: ``sched``, ``TA_SPLIT_PAIRS``, ``ta_layout``), not from the
library's code: the kernel symbol per configuration, the layout (whole rows, causal pairs,
256-row blocks, split, paired split), its grid and the tail variant.  Every described
kernel must exist in the code object the description names, so the query cannot name a
kernel the launch would not find.  The launch entry points plan through the same function
(``plan_launch`` in csrc/tiledattn.cpp), so these tables pin what they launch too.
"""

from __future__ import annotations

import itertools

import pytest

from tiledattention import _lib
from tiledattention.kernels import flash_fwd as ff

CU = 256  # MI355X


@pytest.fixture(scope="module")
def lib():
    if not _lib.library_path().exists():
        pytest.fail("libtiledattn.so is not built: run __graft_entry__.build() first")
    return _lib.load()


@pytest.fixture(scope="module")
def objects():
    return {p.name: p.read_bytes() for p in _lib.code_object_paths()}


def _d(lib, chunk=0, cu=CU, **kw):
    return _lib.describe(lib, _lib.shape_args(**kw), chunk, compute_units=cu)


def _expected_symbol(*, dt, d, tm, tn, causal, tail, accum):
    """The whole-row kernel symbol for a configuration, from the families the code objects
    hold: eight-wave fp32 (128 rows: D <= 160; 64 rows: D 64/96/128/160), eight-wave
    input-dtype (D 64/128, one kernel per TILE_N), four-wave otherwise."""
    c, t = int(causal), int(tail)
    if accum == _lib.TA_ACC_FP32 and tm == 128 and d <= 160:
        return "attn_fwd_pp.hsaco", f"ta_fwd_pp_{dt}_d{d}_c{c}_t{t}"
    if accum == _lib.TA_ACC_FP32 and tm == 64 and d in (64, 96, 128, 160):
        return "attn_fwd_pp.hsaco", f"ta_fwd_pp64_{dt}_d{d}_c{c}_t{t}"
    if accum == _lib.TA_ACC_INPUT and d in (64, 128):
        fam = "ppl" if tm == 128 else "ppl64"
        return "attn_fwd_pp.hsaco", f"ta_fwd_{fam}_n{tn}_{dt}_d{d}_c{c}_t{t}"
    return f"attn_fwd_m{tm}_n{tn}.hsaco", f"ta_fwd_{dt}_d{d}_m{tm}_n{tn}_c{c}_t{t}_a{int(accum)}"


def _configs():
    for dtype, tiles, accum in itertools.product((_lib.TA_FP16, _lib.TA_BF16), _lib.TILE_SHAPES,
                                                 (_lib.TA_ACC_FP32, _lib.TA_ACC_INPUT)):
        for d in (64, 96, 128, 160, 256):
            if d == 96 and accum != _lib.TA_ACC_FP32:
                continue
            if d > 128 and tiles[1] != 64:
                continue
            yield dtype, tiles, accum, d


def _wide_rule(bh, s, d, cu=CU):
    """The wide kernel's rule for a whole-row 64-row tile with fp32 accumulation: D 64 or
    128, 32-row blocks in one round of the CUs, at most two passes (512 keys at D = 128,
    1024 at D = 64), or at most four on more than half the CUs."""
    grid = bh * -(-s // 32)
    passes = -(-s // (512 if d == 128 else 1024))
    return d in (64, 128) and grid <= cu and (passes <= 2 or (passes <= 4 and 2 * grid > cu))


@pytest.mark.parametrize("dtype,tiles,accum,d", list(_configs()))
def test_whole_row_kernel_per_configuration(lib, objects, dtype, tiles, accum, d):
    """One small head (B1 H1: no pairs, no 256-row blocks) at an aligned and a ragged S;
    the symbol and the tail variant follow the families, and the kernel exists.  64-row
    fp32 tiles at D = 64 / 128 run the wide kernel on such grids."""
    dt = "bf16" if dtype == _lib.TA_BF16 else "f16"
    tm, tn = tiles
    eight = (accum == _lib.TA_ACC_FP32 and ((tm == 128 and d <= 160) or (tm == 64 and d in (64, 96, 128, 160)))) \
        or (accum == _lib.TA_ACC_INPUT and d in (64, 128))
    for causal in (False, True):
        for s, aligned in ((512, 1), (512, 0), (320, 1), (300, 1)):
            step = 128 if eight else 1  # the eight-wave kernels step by 128 keys
            tail = not (aligned and s % tm == 0 and s % tn == 0 and s % step == 0)
            desc = _d(lib, S=s, D=d, dtype=dtype, tile_m=tm, tile_n=tn, accum=accum, causal=causal,
                      aligned=aligned)
            f, sym = _expected_symbol(dt=dt, d=d, tm=tm, tn=tn, causal=causal, tail=tail, accum=accum)
            wide = accum == _lib.TA_ACC_FP32 and tm == 64 and _wide_rule(1, s, d)
            if wide:
                f, sym = "attn_fwd_wide.hsaco", f"ta_fwd_wide_{dt}_d{d}_c{int(causal)}_t{int(tail)}"
            assert (desc.code_object.decode(), desc.kernel.decode()) == (f, sym)
            assert desc.kernel + b"\x00" in objects[f], sym
            assert desc.layout == (_lib.TA_LAYOUT_WIDE if wide else _lib.TA_LAYOUT_WHOLE_ROWS)
            assert desc.tail == int(tail)
            rows = 32 if wide else tm
            assert desc.grid == -(-s // rows) and desc.rows == rows
            assert desc.block == (512 if eight else 2 * tm)
            assert desc.in_place_pad == int(eight)
            assert desc.split_capable == int(accum == _lib.TA_ACC_FP32 and d <= 160 and (tm == 128 or d != 256))
            assert desc.merge_kernel == b"" and desc.workspace_bytes == 0


# Causal pairs: the eight-wave kernel (tiles (128, 64) / (128, 128), fp32) at D <= 128,
# two or more query blocks a head, and sched 3, or sched 1 with two or more workgroups per CU.
@pytest.mark.parametrize("kw,pairs", [
    (dict(), True),                                      # C3 S=8192: 512 blocks on 256 CUs
    (dict(S=4096), False),                               # 256 blocks: one wave
    (dict(S=4096, sched=3), True),                       # forced
    (dict(sched=0), False), (dict(sched=2), False),
    (dict(causal=False), False), (dict(D=160), False),
    (dict(accum=_lib.TA_ACC_INPUT), False), (dict(tile_m=64), False),
    (dict(S=128, sched=3), False),                       # one block a head
    (dict(S=8192, H=4, sched=1), False),                 # 256 blocks
    (dict(tile_n=128), True), (dict(D=64), True), (dict(D=96), True),
])
def test_pairing_rule(lib, objects, kw, pairs):
    args = dict(B=1, H=8, S=8192, D=128, causal=True, tile_m=128, tile_n=64, accum=_lib.TA_ACC_FP32,
                sched=1, dtype=_lib.TA_BF16)
    args.update(kw)
    desc = _d(lib, **args)
    nq = -(-args["S"] // args["tile_m"])
    assert (desc.layout == _lib.TA_LAYOUT_PAIRS) is pairs
    if pairs:
        assert desc.kernel.decode() == f"ta_fwd_pp_pair_bf16_d{args['D']}_c1_t0"
        assert desc.grid == args["B"] * args["H"] * ((nq + 1) // 2)
    elif desc.layout == _lib.TA_LAYOUT_ROWS256:  # non-causal B1 H8 S8192: one round of 256 rows
        assert not args["causal"] and _rounds_rule(args["B"], args["H"], args["S"])
        assert desc.grid == args["B"] * args["H"] * -(-args["S"] // 256)
    else:
        assert desc.grid == args["B"] * args["H"] * nq
    assert desc.kernel + b"\x00" in objects[desc.code_object.decode()]


def test_pairing_follows_the_compute_units(lib):
    """The same grid is two waves on 256 CUs (pairs) and one on 512 (whole rows)."""
    kw = dict(B=1, H=8, S=8192, D=128, causal=True, sched=1)
    assert _d(lib, cu=256, **kw).layout == _lib.TA_LAYOUT_PAIRS
    assert _d(lib, cu=512, **kw).layout == _lib.TA_LAYOUT_WHOLE_ROWS
    assert _d(lib, cu=512, **kw).compute_units == 512


# 256-row blocks: non-causal, fp32, tiles (128, 64) / (128, 128), D 64 or 128, when the
# 256-row grid needs at most half the rounds (one workgroup per CU) of the 128-row grid:
# 2 * ceil(B*H*ceil(S/256) / CUs) <= ceil(B*H*ceil(S/128) / CUs).
def _rounds_rule(b, h, s, cu=CU):
    r256 = -(-(b * h * -(-s // 256)) // cu)
    r128 = -(-(b * h * -(-s // 128)) // cu)
    return 2 * r256 <= r128


@pytest.mark.parametrize("kw,rows256", [
    (dict(), True),                                     # C4: 64 heads x 16 blocks = 1024
    (dict(D=64), True), (dict(tile_n=128), True),
    (dict(causal=True), False), (dict(D=160), False), (dict(D=96), False),
    (dict(H=7), True),                                  # 448 blocks: 2 rounds against 4
    (dict(H=6), False),                                 # 384: 2 rounds against 3
    (dict(H=10), False),                                # 640: 3 rounds against 5
    (dict(B=1, H=8, S=8192), True),                     # 256 blocks: 1 round against 2
    (dict(B=1, H=8, S=4096), False),                    # 128: 1 round against 1
    (dict(B=1, H=7, S=8192), True),                     # 224: 1 round against 2
    (dict(B=4, H=16, S=2100), False),                   # 576: 3 rounds against 5
    (dict(accum=_lib.TA_ACC_INPUT), False), (dict(tile_m=64), False),
])
def test_rows256_rule(lib, objects, kw, rows256):
    args = dict(B=4, H=16, S=4096, D=128, causal=False, tile_m=128, tile_n=64, accum=_lib.TA_ACC_FP32,
                sched=1, dtype=_lib.TA_FP16)
    args.update(kw)
    if args["D"] in (64, 128) and not args["causal"] and args["tile_m"] == 128 and args["accum"] == _lib.TA_ACC_FP32:
        assert _rounds_rule(args["B"], args["H"], args["S"]) is rows256
    desc = _d(lib, **args)
    assert (desc.layout == _lib.TA_LAYOUT_ROWS256) is rows256
    if rows256:
        assert desc.kernel.decode() == f"ta_fwd_pp256_f16_d{args['D']}_c0_t{int(args['S'] % 256 != 0)}"
        assert desc.grid == args["B"] * args["H"] * -(-args["S"] // 256) and desc.rows == 256
    assert desc.kernel + b"\x00" in objects[desc.code_object.decode()]


def test_rows256_rule_follows_the_compute_units(lib):
    """The same grid is one round of 256-row blocks on 256 CUs, half a round on 512."""
    kw = dict(B=1, H=8, S=8192, D=128, causal=False)
    assert _d(lib, cu=256, **kw).layout == _lib.TA_LAYOUT_ROWS256
    assert _d(lib, cu=512, **kw).layout == _lib.TA_LAYOUT_WHOLE_ROWS


def test_rows256_tail_variant_when_s_is_not_a_multiple_of_256(lib):
    desc = _d(lib, B=4, H=15, S=4224, D=128, causal=False)  # 128-aligned, not 256
    assert desc.layout == _lib.TA_LAYOUT_ROWS256
    assert desc.tail == 1 and desc.kernel.decode() == "ta_fwd_pp256_bf16_d128_c0_t1"
    assert desc.grid == 60 * 17


@pytest.mark.parametrize("d", [64, 96, 128, 160])
@pytest.mark.parametrize("causal", [False, True])
def test_split_descriptions(lib, objects, d, causal):
    """Chunks of 2 steps at S=1000 (8 blocks, 8 key steps): split kernel + merge kernel,
    both in the eight-wave object, a workspace, the kernel's tail variant (S ragged)."""
    desc = _d(lib, 2, B=1, H=2, S=1000, D=d, causal=causal)
    assert desc.layout == _lib.TA_LAYOUT_SPLIT and desc.chunk_steps == 2
    assert desc.kernel.decode() == f"ta_fwd_pp_split_bf16_d{d}_c{int(causal)}_t1"
    assert desc.merge_kernel.decode() == f"ta_fwd_merge_bf16_d{d}_c{int(causal)}"
    assert desc.block == 512 and desc.merge_block > 0 and desc.merge_grid > 0
    assert desc.workspace_bytes > 0
    # 8 blocks, chunks of 2: up to 4 chunks a block, 2 x 6 (causal) or 2 x 8 split blocks,
    # far below 3/8 of the CUs: the merge kernel runs
    assert desc.merge_in_kernel == 0
    need = __import__("ctypes").c_int64(0)
    a = _lib.shape_args(B=1, H=2, S=1000, D=d, causal=causal)
    assert lib.ta_split_workspace_size(__import__("ctypes").byref(a), 2, __import__("ctypes").byref(need)) == 0
    assert need.value == desc.workspace_bytes
    for sym in (desc.kernel, desc.merge_kernel):
        assert sym + b"\x00" in objects["attn_fwd_pp.hsaco"], sym


@pytest.mark.parametrize("kw,chunk,mik", [
    # the paired split: two chunks a block
    (dict(B=1, H=8, S=4096, causal=True), _lib.TA_SPLIT_PAIRS, 1),
    (dict(B=1, H=1, S=4096, causal=True), _lib.TA_SPLIT_PAIRS, 1),
    # at most two chunks a block, any grid
    (dict(B=1, H=1, S=2048, causal=True), 8, 1),        # 16 blocks: 8 split in 2
    (dict(B=1, H=2, S=4096, causal=False), 16, 1),      # 32 steps in 2 chunks
    # more chunks: only with 3/8 of the CUs' worth of split blocks (96 of 256)
    (dict(B=1, H=8, S=2048, causal=True), 4, 1),        # 8 x 12 = 96 split blocks, 4 chunks
    (dict(B=1, H=4, S=4096, causal=True), 11, 0),       # 4 x 21 = 84, 3 chunks
    (dict(B=1, H=1, S=4096, causal=True), 5, 0),        # 27, 7 chunks
    (dict(B=1, H=1, S=2048, causal=False), 4, 0),       # 16, 4 chunks
    (dict(B=1, H=8, S=4096, causal=True), 1, 1),        # 8 x 31 = 248 split blocks
    # more partial slots than a counter region (16384) holds: the merge kernel
    (dict(B=4, H=16, S=4096, causal=True), 1, 0),       # 64 heads x 496 slots
])
def test_in_kernel_merge_rule(lib, kw, chunk, mik):
    """The split kernel merges its own blocks (the last workgroup of a block combines its
    partials; a counter per block, its chunk-0 slot) when the counters fit a region and no
    block has more than two chunks or the split blocks number 3/8 of the CUs or more;
    otherwise the merge kernel runs after it."""
    desc = _d(lib, chunk, D=128, **kw)
    assert desc.layout in (_lib.TA_LAYOUT_SPLIT, _lib.TA_LAYOUT_PAIRED_SPLIT)
    assert desc.merge_in_kernel == mik and desc.merge_grid > 0 and desc.merge_kernel != b""


def test_in_kernel_merge_rule_follows_the_compute_units(lib):
    kw = dict(B=1, H=8, S=2048, D=128, causal=True)  # 96 split blocks of up to 4 chunks
    assert _d(lib, 4, cu=256, **kw).merge_in_kernel == 1
    assert _d(lib, 4, cu=512, **kw).merge_in_kernel == 0
    whole = _d(lib, 0, B=1, H=8, S=4096, D=128, causal=True)
    assert whole.merge_in_kernel == 0 and whole.merge_kernel == b""


def test_paired_split_and_chunks_that_split_nothing(lib):
    desc = _d(lib, _lib.TA_SPLIT_PAIRS, B=1, H=8, S=4096, D=128, causal=True)
    assert desc.layout == _lib.TA_LAYOUT_PAIRED_SPLIT and desc.chunk_steps == _lib.TA_SPLIT_PAIRS
    assert desc.kernel.decode() == "ta_fwd_pp_psplit_bf16_d128_c1_t0"
    assert desc.grid == 8 * 32  # the whole-row grid's size
    # a chunk at least as long as every row splits nothing: whole rows, no workspace
    whole = _d(lib, 64, B=1, H=8, S=4096, D=128, causal=True)
    assert whole.layout == _lib.TA_LAYOUT_WHOLE_ROWS and whole.workspace_bytes == 0
    # the paired split of a non-causal call is the whole-row launch
    assert _d(lib, _lib.TA_SPLIT_PAIRS, B=1, H=8, S=4096, D=128).layout == _lib.TA_LAYOUT_WHOLE_ROWS


def test_split_on_a_configuration_without_split_kernels(lib):
    with pytest.raises(ValueError, match="TA_EUNSUPPORTED"):
        _d(lib, 2, S=1000, D=128, tile_m=64, accum=_lib.TA_ACC_INPUT)
    with pytest.raises(ValueError, match="TA_EUNSUPPORTED"):  # the paired split: 128-row tiles
        _d(lib, _lib.TA_SPLIT_PAIRS, S=8192, D=128, tile_m=64, causal=True)
    # ... unless the chunk splits nothing, which runs whole rows on any kernel
    assert _d(lib, 64, S=1000, D=128, tile_m=64, accum=_lib.TA_ACC_INPUT).layout == _lib.TA_LAYOUT_WHOLE_ROWS


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d", [64, 96, 128, 160])
def test_64_row_split_descriptions(lib, objects, d, causal):
    """Chunks on the 64-row kernel: the 128-row numbering with two 64-row halves per item
    (twice the workgroups of the 128-row split), the same merge kernel and workspace."""
    d128 = _d(lib, 2, B=1, H=2, S=1000, D=d, causal=causal)
    d64 = _d(lib, 2, B=1, H=2, S=1000, D=d, causal=causal, tile_m=64)
    assert d64.layout == _lib.TA_LAYOUT_SPLIT and d64.rows == 64
    assert d64.kernel.decode() == f"ta_fwd_pp64_split_bf16_d{d}_c{int(causal)}_t1"
    assert d64.grid == 2 * d128.grid
    assert (d64.merge_kernel, d64.merge_grid, d64.workspace_bytes) == (
        d128.merge_kernel, d128.merge_grid, d128.workspace_bytes)
    for sym in (d64.kernel, d64.merge_kernel):
        assert sym + b"\x00" in objects["attn_fwd_pp.hsaco"], sym
    # the dispatch model plans the 128-row kernel only: auto leaves 64-row tiles whole
    plan = lib.ta_split_plan_model(1000, 2, int(causal), 256)
    a = _lib.shape_args(B=1, H=2, S=1000, D=d, causal=causal, tile_m=64)
    out = __import__("ctypes").c_int32(-7)
    assert lib.ta_split_plan(__import__("ctypes").byref(a), __import__("ctypes").byref(out)) in (0, 4)
    assert plan >= 0


def test_zero_size_and_invalid_requests(lib):
    desc = _d(lib, S=0)
    assert desc.grid == 0 and desc.kernel == b""
    with pytest.raises(ValueError, match="head_dim"):
        _d(lib, D=80)
    with pytest.raises(ValueError, match="compute_units"):
        _d(lib, cu=0)
    with pytest.raises(ValueError, match="chunk_steps"):
        _d(lib, -5)


def test_policy_defaults_run_the_described_kernels(lib):
    """The host policy's default tiles for the BASELINE configurations, through the library:
    C1 64-row tile on the wide kernel (tail variant: S = 64 is not a whole 128-key step), C2
    (64, 64) non-causal and C3 S = 512 the wide kernel (32-row blocks in one round of the
    CUs), C3 S = 2048 the 64-row kernel (512 blocks of 32 rows would be two rounds), S = 4096
    whole 128-row blocks, S=8192 causal pairs, C4 256-row blocks, C5 causal pairs."""
    cases = [
        ((1, 2, 64, 64), True, "ta_fwd_wide_f16_d64_c1_t1", _lib.TA_LAYOUT_WIDE, _lib.TA_FP16),
        ((1, 8, 1024, 64), False, "ta_fwd_wide_f16_d64_c0_t0", _lib.TA_LAYOUT_WIDE, _lib.TA_FP16),
        ((1, 8, 512, 128), True, "ta_fwd_wide_bf16_d128_c1_t0", _lib.TA_LAYOUT_WIDE, _lib.TA_BF16),
        ((1, 8, 1024, 128), True, "ta_fwd_wide_bf16_d128_c1_t0", _lib.TA_LAYOUT_WIDE, _lib.TA_BF16),
        ((1, 8, 2048, 128), True, "ta_fwd_pp64_bf16_d128_c1_t0", _lib.TA_LAYOUT_WHOLE_ROWS, _lib.TA_BF16),
        ((1, 8, 4096, 128), True, "ta_fwd_pp_bf16_d128_c1_t0", _lib.TA_LAYOUT_WHOLE_ROWS, _lib.TA_BF16),
        ((1, 8, 8192, 128), True, "ta_fwd_pp_pair_bf16_d128_c1_t0", _lib.TA_LAYOUT_PAIRS, _lib.TA_BF16),
        ((4, 16, 4096, 128), False, "ta_fwd_pp256_bf16_d128_c0_t0", _lib.TA_LAYOUT_ROWS256, _lib.TA_BF16),
        ((4, 16, 4096, 64), False, "ta_fwd_pp256_f16_d64_c0_t0", _lib.TA_LAYOUT_ROWS256, _lib.TA_FP16),
        ((1, 8, 16384, 128), True, "ta_fwd_pp_pair_f16_d128_c1_t0", _lib.TA_LAYOUT_PAIRS, _lib.TA_FP16),
    ]
    for (b, h, s, d), causal, kernel, layout, dtype in cases:
        tm, tn = ff._default_tile_config_for_shape_gfx950(seq_len=s, head_dim=d, causal=causal, n_bh=b * h,
                                                          compute_units=CU)
        if (b, h, s, d) == (1, 8, 1024, 64):
            tm, tn = 64, 64  # C2 pins its tile
        n_qblk = -(-s // tm)
        sched = ff._resolve_sched(n_blocks=b * h * n_qblk, causal=causal, tile_m=tm, tile_n=tn,
                                  head_dim=d, compute_units=CU)
        desc = _d(lib, B=b, H=h, S=s, D=d, causal=causal, tile_m=tm, tile_n=tn, sched=sched, dtype=dtype)
        assert (desc.kernel.decode(), desc.layout) == (kernel, layout), (b, h, s, d)
