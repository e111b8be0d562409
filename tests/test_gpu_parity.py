"""GPU parity of the gfx950 SDPA forward against the CPU oracle, at every BASELINE config.

Every case names itself on stdout before touching the GPU.  Inputs come from the CPU
generator (oracle.make_inputs), so they are bit-identical to what the oracle sees.  Sizes
the oracle finishes in seconds are compared in full; the long sequences (S >= 4096) are
compared on sampled query rows (first/last 64 rows plus random rows), which the oracle
computes exactly and independently of the other rows.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.parity_util import (
    LOWP_TOL,
    TOL,
    as_f32,
    check_close,
    inputs,
    kernel_for,
    knobs,
    oracle_f32,
    run_gpu,
    sample_rows,
    say,
)

pytestmark = pytest.mark.gpu

TILES = [(64, 64), (64, 128), (128, 64), (128, 128)]


# ---------------------------------------------------------------- BASELINE configs

def test_c1_example_workload_all_tiles(gpu):
    """C1: B1 H2 S64 D64 fp16 causal, seed 0 (the reference's example.py:19-24 workload)."""
    q, k, v = inputs((1, 2, 64, 64), "float16", 0)
    ref = oracle_f32(q, k, v, causal=True)
    for tm, tn in [(None, None)] + TILES:
        say(f"C1 fp16 causal (1,2,64,64) seed=0 tiles={(tm, tn) if tm else 'default'}")
        env = {} if tm is None else {"tile_m": tm, "tile_n": tn}
        out = run_gpu(q, k, v, causal=True, **env)
        assert out.shape == (1, 2, 64, 64) and out.dtype == q.dtype
        check_close(as_f32(out), ref, "float16", what=f"C1 tiles={tm},{tn}")


def test_reference_small_noncausal_vs_torch(gpu):
    """Port of the reference's GPU test (tests/test_sdpa_correctness_small.py:20-44):
    (1,2,64,64) fp16 non-causal, seed 0, against torch's SDPA at atol=rtol=2.5e-2; the
    torch result is computed in float32 from the same inputs."""
    import torch

    say("reference small test (1,2,64,64) fp16 non-causal seed=0 vs torch SDPA")
    q, k, v = inputs((1, 2, 64, 64), "float16", 0)
    out = run_gpu(q, k, v, causal=False)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.float().cuda(), k.float().cuda(), v.float().cuda(), attn_mask=None, dropout_p=0.0, is_causal=False
    ).to(torch.float16)
    torch.cuda.synchronize()
    assert out.shape == ref.shape
    assert out.dtype == ref.dtype
    assert torch.allclose(out, ref, atol=2.5e-2, rtol=2.5e-2)
    check_close(as_f32(out), oracle_f32(q, k, v, causal=False), "float16", what="reference small")


def test_c2_fp16_noncausal_s1024_d64(gpu):
    """C2: B1 H8 S1024 D64 fp16 non-causal, tile 64x64, fp32 accumulation, seed 2026."""
    q, k, v = inputs((1, 8, 1024, 64), "float16", 2026)
    ref = oracle_f32(q, k, v, causal=False)
    say("C2 fp16 non-causal (1,8,1024,64) seed=2026 tile 64x64 accum fp32")
    out = run_gpu(q, k, v, causal=False, tile_m=64, tile_n=64, accum_mode="fp32")
    check_close(as_f32(out), ref, "float16", what="C2")
    say("C2 with default knobs (auto accumulation: fp32 on gfx950)")
    out = run_gpu(q, k, v, causal=False)
    check_close(as_f32(out), ref, "float16", what="C2 default")
    say("C2 with the reference's auto choice for this shape (input-dtype accumulation)")
    out = run_gpu(q, k, v, causal=False, accum_mode="fp16")
    check_close(as_f32(out), ref, "float16", tol=LOWP_TOL["float16"], what="C2 accum fp16")


@pytest.mark.parametrize("s", [512, 1024, 2048, 4096, 8192])
def test_c3_bf16_causal_d128(gpu, s):
    """C3: B1 H8 D128 bf16 causal, seed 1234, S swept; S >= 4096 on sampled rows."""
    q, k, v = inputs((1, 8, s, 128), "bfloat16", 1234)
    rows = None if s <= 2048 else sample_rows(s, 192)
    ref = oracle_f32(q, k, v, causal=True, rows=rows)
    say(f"C3 bf16 causal (1,8,{s},128) seed=1234 default tiles rows={'all' if rows is None else len(rows)}")
    out = run_gpu(q, k, v, causal=True)
    check_close(as_f32(out, rows), ref, "bfloat16", what=f"C3 S={s}")
    if s <= 2048:
        for tm, tn in TILES:
            say(f"C3 bf16 causal S={s} tiles=({tm},{tn})")
            out = run_gpu(q, k, v, causal=True, tile_m=tm, tile_n=tn)
            check_close(as_f32(out), ref, "bfloat16", what=f"C3 S={s} tiles={tm},{tn}")


@pytest.mark.parametrize("dtype,causal,d,s", [
    ("float16", False, 128, 8192),   # the reference's headline curve (benchmark_results.csv:128)
    ("float16", False, 128, 2048),
    ("bfloat16", False, 128, 8192),
    ("float16", False, 64, 8192), ("bfloat16", False, 64, 8192),
    ("float16", True, 64, 8192), ("bfloat16", True, 64, 8192),
    ("float16", False, 64, 1024), ("bfloat16", True, 64, 2048),
])
def test_metric_grid_b1_h8(gpu, dtype, causal, d, s):
    """The bench's grid workloads (B1 H8, seed 1234, default knobs): the metric's other
    curves, non-causal D = 128 and D = 64 both ways, against the oracle (sampled rows for
    S >= 4096, with every output element checked for finiteness)."""
    q, k, v = inputs((1, 8, s, d), dtype, 1234)
    rows = None if s <= 2048 else sample_rows(s, 128)
    ref = oracle_f32(q, k, v, causal=causal, rows=rows)
    say(f"grid {dtype} causal={causal} (1,8,{s},{d}) seed=1234 rows={'all' if rows is None else len(rows)}")
    out = run_gpu(q, k, v, causal=causal)
    check_close(as_f32(out, rows), ref, dtype, what=f"grid {dtype} causal={causal} S={s} D={d}")


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("d", [64, 128])
def test_c4_noncausal_tile_sweep(gpu, dtype, d):
    """C4: B4 H16 S4096 non-causal, inputs N(0,1)*0.5, seed 2026, TILE_M/TILE_N in {64,128}."""
    q, k, v = inputs((4, 16, 4096, d), dtype, 2026, scale_inputs=0.5)
    rows = sample_rows(4096, 64)
    ref = oracle_f32(q, k, v, causal=False, rows=rows)
    for tm, tn in TILES:
        say(f"C4 {dtype} non-causal (4,16,4096,{d}) seed=2026 tiles=({tm},{tn}) accum fp32")
        out = run_gpu(q, k, v, causal=False, tile_m=tm, tile_n=tn, accum_mode="fp32")
        check_close(as_f32(out, rows), ref, dtype, what=f"C4 {dtype} D={d} tiles={tm},{tn}")


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("d", [64, 128])
def test_c4_input_dtype_accumulation(gpu, dtype, d):
    """C4 with ACCUM_MODE=fp16 (flash_fwd.py:301-372) at every tile: 32-64 roundings of O
    per key slice, sampled rows against the fp32 oracle at the input-dtype bound."""
    q, k, v = inputs((4, 16, 4096, d), dtype, 2026, scale_inputs=0.5)
    rows = sample_rows(4096, 64)
    ref = oracle_f32(q, k, v, causal=False, rows=rows)
    for tm, tn in TILES:
        say(f"C4 {dtype} non-causal (4,16,4096,{d}) seed=2026 tiles=({tm},{tn}) accum fp16")
        out = run_gpu(q, k, v, causal=False, tile_m=tm, tile_n=tn, accum_mode="fp16")
        check_close(as_f32(out, rows), ref, dtype, tol=LOWP_TOL[dtype],
                    what=f"C4 {dtype} D={d} tiles={tm},{tn} accum fp16")


@pytest.mark.parametrize("tiles", [(None, None), (64, 128)])
def test_c5_input_dtype_accumulation(gpu, tiles):
    """C5 (S = 16384, fp16, causal) with ACCUM_MODE=fp16: up to 128 roundings of O per key
    slice at TILE_N = 64, sampled rows (the last ones see every key) against the oracle."""
    tm, tn = tiles
    q, k, v = inputs((1, 8, 16384, 128), "float16", 1234)
    rows = sample_rows(16384, 128)
    ref = oracle_f32(q, k, v, causal=True, rows=rows)
    say(f"C5 fp16 causal (1,8,16384,128) seed=1234 tiles=({tm},{tn}) accum fp16 rows={len(rows)}")
    out = run_gpu(q, k, v, causal=True, tile_m=tm, tile_n=tn, accum_mode="fp16")
    check_close(as_f32(out, rows), ref, "float16", tol=LOWP_TOL["float16"], what=f"C5 accum fp16 tiles={tm},{tn}")


@pytest.mark.parametrize("outliers", [False, True])
def test_c5_long_sequence_causal(gpu, outliers):
    """C5: B1 H8 S16384 D128 fp16 causal, seed 1234; C5b: 1% of k entries x20 (seed 1235)."""
    kw = dict(outlier_frac=0.01, outlier_gain=20.0, outlier_seed=1235) if outliers else {}
    q, k, v = inputs((1, 8, 16384, 128), "float16", 1234, **kw)
    rows = sample_rows(16384, 128)
    ref = oracle_f32(q, k, v, causal=True, rows=rows)
    say(f"C5{'b' if outliers else ''} fp16 causal (1,8,16384,128) seed=1234 rows={len(rows)}")
    out = run_gpu(q, k, v, causal=True)
    check_close(as_f32(out, rows), ref, "float16", what=f"C5{'b' if outliers else ''}")


# ---------------------------------------------------------------- ragged / edge shapes

@pytest.mark.parametrize("s", [1, 17, 100, 1000])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype,d", [("float16", 64), ("bfloat16", 128)])
def test_tails_all_tiles(gpu, s, causal, dtype, d):
    """S not a multiple of the tile: masked tails (flash_fwd.py:400-403, 415-423)."""
    q, k, v = inputs((2, 3, s, d), dtype, 100 + s)
    ref = oracle_f32(q, k, v, causal=causal)
    for tm, tn in TILES:
        say(f"tail {dtype} (2,3,{s},{d}) causal={causal} tiles=({tm},{tn})")
        out = run_gpu(q, k, v, causal=causal, tile_m=tm, tile_n=tn, accum_mode="fp32")
        check_close(as_f32(out), ref, dtype, what=f"tail S={s} tiles={tm},{tn}")


@pytest.mark.parametrize("d", [8, 32, 48, 80, 96, 100])
def test_head_dim_padding(gpu, d):
    """D outside {64,128}: a multiple of 8 runs in place on the eight-wave kernels (every
    tile, fp32 or input-dtype accumulation), whose missing columns read as zero (dense
    output of width D); other D are zero-padded on the host and the output is a sliced
    view."""
    q, k, v = inputs((1, 2, 200, d), "float16", 7 + d)
    for causal in (False, True):
        ref = oracle_f32(q, k, v, causal=causal)
        say(f"pad fp16 (1,2,200,{d}) causal={causal} default tile")
        out = run_gpu(q, k, v, causal=causal)
        assert out.shape == (1, 2, 200, d)
        assert out.is_contiguous() == (d % 8 == 0)
        check_close(as_f32(out), ref, "float16", what=f"pad D={d}")
        say(f"pad fp16 (1,2,200,{d}) causal={causal} tile 64x64 (64-row eight-wave kernel)")
        out = run_gpu(q, k, v, causal=causal, tile_m=64, tile_n=64)
        assert out.shape == (1, 2, 200, d) and out.is_contiguous() == (d % 8 == 0)
        check_close(as_f32(out), ref, "float16", what=f"64-row pad D={d}")
        say(f"pad fp16 (1,2,200,{d}) causal={causal} tile 64x64 input-dtype accumulation")
        low = run_gpu(q, k, v, causal=causal, tile_m=64, tile_n=64, accum_mode="fp16")
        assert low.shape == (1, 2, 200, d) and low.is_contiguous() == (d % 8 == 0)
        check_close(as_f32(low), ref, "float16", tol=LOWP_TOL["float16"], what=f"input-dtype pad D={d}")


@pytest.mark.parametrize("d,dtype,causal,s", [
    (96, "bfloat16", True, 1000), (120, "float16", False, 777), (56, "bfloat16", False, 1500),
    (72, "float16", True, 2048), (104, "bfloat16", True, 4096),
])
def test_head_dim_in_kernel_padding(gpu, d, dtype, causal, s):
    """Narrower head dims on the eight-wave kernel without host copies: ragged S, both
    dtypes, split key ranges, [B,S,H,D]-strided views (row stride H*D, not a multiple of the
    kernel's D), all against the oracle."""
    import torch

    from tiledattention import sdpa

    q, k, v = inputs((2, 3, s, d), dtype, 40 + d)
    rows = None if s <= 2048 else sample_rows(s, 96)
    ref = oracle_f32(q, k, v, causal=causal, rows=rows)
    say(f"in-kernel pad {dtype} (2,3,{s},{d}) causal={causal}")
    out = run_gpu(q, k, v, causal=causal)
    assert out.shape == (2, 3, s, d) and out.is_contiguous()
    check_close(as_f32(out, rows), ref, dtype, what=f"in-kernel pad D={d}")
    say(f"in-kernel pad {dtype} (2,3,{s},{d}) causal={causal} split=2")
    out = run_gpu(q, k, v, causal=causal, split=2)
    check_close(as_f32(out, rows), ref, dtype, what=f"in-kernel pad D={d} split")
    dev = torch.device("cuda:0")
    bshd = [t.transpose(1, 2).contiguous().to(dev).transpose(1, 2) for t in (q, k, v)]
    say(f"in-kernel pad {dtype} (2,3,{s},{d}) causal={causal} [B,S,H,D] views")
    out = sdpa(*bshd, causal=causal)
    torch.cuda.synchronize()
    check_close(as_f32(out, rows), ref, dtype, what=f"in-kernel pad D={d} BSHD")


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("d", [160, 256])
@pytest.mark.parametrize("tiles", [(None, None), (64, 64), (128, 64)])
def test_wide_head_dims(gpu, dtype, d, tiles):
    """Native D = 160 / 256 kernels (64-key tiles), causal and not, a ragged length."""
    q, k, v = inputs((1, 2, 300, d), dtype, 1000 + d)
    tm, tn = tiles
    for causal in (False, True):
        say(f"wide D={d} {dtype} (1,2,300,{d}) causal={causal} tiles=({tm},{tn})")
        out = run_gpu(q, k, v, causal=causal, tile_m=tm, tile_n=tn)
        assert out.shape == (1, 2, 300, d)
        check_close(as_f32(out), oracle_f32(q, k, v, causal=causal), dtype, what=f"D={d}")


@pytest.mark.parametrize("d,dtype,causal,s", [
    (160, "bfloat16", True, 2048), (160, "float16", False, 1000), (152, "bfloat16", False, 777),
    (136, "float16", True, 3000),
])
def test_eight_wave_d160(gpu, d, dtype, causal, s):
    """Kernel head dim 160 on the 128-row eight-wave kernel (tile (128, 64); these grids'
    default is 64 rows where their 64-row blocks fit the CUs once): stages split into a
    128-column part and a 32-column tail part; head dims 129-159 run in place with the
    missing tail columns read as zero.  Ragged S, both dtypes, [B,S,H,D] views."""
    import torch

    from tiledattention import sdpa

    q, k, v = inputs((2, 3, s, d), dtype, 160 + d + s)
    assert kernel_for(q, k, v, causal=causal, tile_m=128, tile_n=64).startswith("ta_fwd_pp_")
    rows = None if s <= 2048 else sample_rows(s, 96)
    ref = oracle_f32(q, k, v, causal=causal, rows=rows)
    say(f"eight-wave D={d} {dtype} (2,3,{s},{d}) causal={causal}")
    out = run_gpu(q, k, v, causal=causal, tile_m=128, tile_n=64)
    assert out.shape == (2, 3, s, d) and out.is_contiguous()
    check_close(as_f32(out, rows), ref, dtype, what=f"eight-wave D={d}")
    dev = torch.device("cuda:0")
    bshd = [t.transpose(1, 2).contiguous().to(dev).transpose(1, 2) for t in (q, k, v)]
    say(f"eight-wave D={d} {dtype} (2,3,{s},{d}) causal={causal} [B,S,H,D] views")
    with knobs(tile_m=128, tile_n=64):
        out = sdpa(*bshd, causal=causal)
    torch.cuda.synchronize()
    check_close(as_f32(out, rows), ref, dtype, what=f"eight-wave D={d} BSHD")
    say(f"default tile D={d} {dtype} (2,3,{s},{d}) causal={causal}")
    out = run_gpu(q, k, v, causal=causal)
    check_close(as_f32(out, rows), ref, dtype, what=f"default tile D={d}")


@pytest.mark.parametrize("d,dtype,causal,s,tn", [
    (160, "bfloat16", True, 2048, 64), (160, "float16", False, 1000, 64), (144, "bfloat16", True, 777, 64),
    (136, "float16", False, 3000, 64), (160, "bfloat16", True, 1, 64), (160, "float16", True, 129, 64),
])
def test_64_row_d160(gpu, d, dtype, causal, s, tn):
    """Kernel head dim 160 on the 64-row eight-wave kernel (tile (64, 64), the only TILE_N
    above D = 128; fp32 accumulation): the 128 + 32 column stage split, five 32-wide d blocks of O and the
    four-way merge of five chunks a part; head dims 129-159 in place.  Ragged S, both
    dtypes, [B,S,H,D] views."""
    import torch

    from tiledattention import sdpa

    q, k, v = inputs((2, 3, s, d), dtype, 640 + d + s)
    assert kernel_for(q, k, v, causal=causal, tile_m=64, tile_n=tn).startswith("ta_fwd_pp64_")
    rows = None if s <= 2048 else sample_rows(s, 96)
    ref = oracle_f32(q, k, v, causal=causal, rows=rows)
    say(f"64-row D={d} {dtype} (2,3,{s},{d}) causal={causal} tile (64,{tn})")
    out = run_gpu(q, k, v, causal=causal, tile_m=64, tile_n=tn, accum_mode="fp32")
    assert out.shape == (2, 3, s, d) and out.is_contiguous()
    check_close(as_f32(out, rows), ref, dtype, what=f"64-row D={d}")
    dev = torch.device("cuda:0")
    bshd = [t.transpose(1, 2).contiguous().to(dev).transpose(1, 2) for t in (q, k, v)]
    say(f"64-row D={d} {dtype} (2,3,{s},{d}) causal={causal} [B,S,H,D] views")
    with knobs(tile_m=64, tile_n=tn, accum_mode="fp32"):
        out = sdpa(*bshd, causal=causal)
    torch.cuda.synchronize()
    check_close(as_f32(out, rows), ref, dtype, what=f"64-row D={d} BSHD")


@pytest.mark.parametrize("d,dtype,causal,s,tn", [
    (96, "bfloat16", True, 2048, 64), (96, "float16", False, 1000, 128), (88, "bfloat16", False, 777, 64),
    (72, "float16", True, 3000, 64), (80, "bfloat16", True, 128, 128), (96, "float16", True, 1, 64),
])
def test_eight_wave_d96(gpu, d, dtype, causal, s, tn):
    """Kernel head dim 96 on the eight-wave kernels with fp32 accumulation: stages split
    into a 64-column main part and a 32-column tail part, three 32-wide d blocks of O (the
    odd-block merge at 128 rows, the four-way merge of three chunks a part at 64 rows); head
    dims 65-95 run in place with the missing columns read as zero.  Ragged S, both dtypes,
    both row counts, [B,S,H,D] views, split key ranges (one-step chunks) and, causal,
    query-block pairs."""
    import torch

    from tiledattention import _lib, sdpa
    from tiledattention.kernels import flash_fwd as ff

    q, k, v = inputs((2, 3, s, d), dtype, 96 + d + s)
    rows = None if s <= 2048 else sample_rows(s, 96)
    ref = oracle_f32(q, k, v, causal=causal, rows=rows)
    say(f"eight-wave D={d} -> 96 {dtype} (2,3,{s},{d}) causal={causal} tile (128,{tn})")
    out = run_gpu(q, k, v, causal=causal, tile_m=128, tile_n=tn)
    assert out.shape == (2, 3, s, d) and out.is_contiguous()
    check_close(as_f32(out, rows), ref, dtype, what=f"eight-wave D={d} on the D=96 kernel")
    assert any(pl.args is not None and _lib.FwdArgs.from_buffer_copy(pl.args).D == 96
               for pl in ff._PLANS.values() if not pl.empty)
    dev = torch.device("cuda:0")
    bshd = [t.transpose(1, 2).contiguous().to(dev).transpose(1, 2) for t in (q, k, v)]
    say(f"eight-wave D={d} -> 96 {dtype} (2,3,{s},{d}) causal={causal} [B,S,H,D] views")
    with knobs(tile_m=128, tile_n=tn):
        out = sdpa(*bshd, causal=causal)
    torch.cuda.synchronize()
    check_close(as_f32(out, rows), ref, dtype, what=f"eight-wave D={d} BSHD")
    say(f"64-row D={d} -> 96 {dtype} (2,3,{s},{d}) causal={causal} tile (64,{tn})")
    out = run_gpu(q, k, v, causal=causal, tile_m=64, tile_n=tn)
    check_close(as_f32(out, rows), ref, dtype, what=f"64-row D={d} on the D=96 kernel")
    say(f"eight-wave D={d} -> 96 {dtype} (2,3,{s},{d}) causal={causal} split=1")
    out = run_gpu(q, k, v, causal=causal, tile_m=128, tile_n=tn, split=1)
    check_close(as_f32(out, rows), ref, dtype, what=f"eight-wave D={d} split")
    if causal:
        say(f"eight-wave D={d} -> 96 {dtype} (2,3,{s},{d}) causal pairs (sched 3)")
        out = run_gpu(q, k, v, causal=True, tile_m=128, tile_n=tn, sched=3, split="off")
        check_close(as_f32(out, rows), ref, dtype, what=f"eight-wave D={d} pairs")


@pytest.mark.parametrize("tn", [64, 128])
@pytest.mark.parametrize("s,causal,dtype", [
    (64, True, "float16"), (100, False, "bfloat16"), (320, True, "bfloat16"), (448, False, "float16"),
    (1000, True, "float16"), (1536, False, "bfloat16"),
])
def test_eight_wave_64_row_tiles(gpu, tn, s, causal, dtype):
    """Tiles (64, tn) with fp32 accumulation run the 64-row eight-wave kernel (four key
    slices per row block, merged at the end): lengths that are multiples of 64 but not of
    the 128-key step (320, 448: the tail-masked variant), ragged ones, D = 64 and 128, and
    narrower head dims padded in place (D = 48 and 96); [B,S,H,D] views for one case.  The
    heads are enough that 32-row blocks would need a second round of the CUs: smaller grids
    run the wide kernel at D = 64 and 128 (tests/test_gpu_wide.py)."""
    import torch

    from tiledattention import sdpa

    h = max(3, 256 // (2 * -(-s // 32)) + 1)
    for d in (64, 128, 48, 96):
        q, k, v = inputs((2, h, s, d), dtype, 6400 + s + d + tn)
        assert kernel_for(q, k, v, causal=causal, tile_m=64, tile_n=tn).startswith("ta_fwd_pp64_")
        say(f"64-row eight-wave {dtype} (2,{h},{s},{d}) causal={causal} tiles=(64,{tn})")
        out = run_gpu(q, k, v, causal=causal, tile_m=64, tile_n=tn)
        assert out.shape == (2, h, s, d)
        ref = oracle_f32(q, k, v, causal=causal)
        check_close(as_f32(out), ref, dtype, what=f"64-row D={d}")
        if d == 96 and s == 1000:
            dev = torch.device("cuda:0")
            bshd = [t.transpose(1, 2).contiguous().to(dev).transpose(1, 2) for t in (q, k, v)]
            say(f"64-row eight-wave {dtype} (2,{h},{s},{d}) [B,S,H,D] views")
            from tests.parity_util import knobs
            with knobs(tile_m=64, tile_n=tn):
                out = sdpa(*bshd, causal=causal)
            torch.cuda.synchronize()
            check_close(as_f32(out), ref, dtype, what="64-row BSHD")


@pytest.mark.parametrize("d", [144, 200])
def test_wide_head_dim_padding(gpu, d):
    """D in (128, 256] outside {160, 256}: padded to the next wide kernel."""
    q, k, v = inputs((2, 1, 257, d), "bfloat16", 2000 + d)
    for causal in (False, True):
        say(f"wide pad bf16 (2,1,257,{d}) causal={causal}")
        out = run_gpu(q, k, v, causal=causal)
        check_close(as_f32(out), oracle_f32(q, k, v, causal=causal), "bfloat16", what=f"pad D={d}")


def test_wide_head_dim_input_dtype_accumulation(gpu):
    q, k, v = inputs((1, 2, 256, 160), "float16", 3160)
    say("wide D=160 fp16 accumulation (1,2,256,160) causal")
    out = run_gpu(q, k, v, causal=True, accum_mode="fp16")
    check_close(as_f32(out), oracle_f32(q, k, v, causal=True), "float16", tol=LOWP_TOL["float16"],
                what="D=160 fp16 accum")


@pytest.mark.parametrize("tiles", [(None, None), (64, 64)])
@pytest.mark.parametrize("s,causal,dtype", [
    (512, False, "bfloat16"), (512, True, "float16"), (1000, False, "float16"), (1536, True, "bfloat16"),
])
def test_d256_direct_staging(gpu, tiles, s, causal, dtype):
    """D = 256 kernels load K/V tiles straight into LDS (swizzled rows; the 64-row tiles
    refill K and V separately through one stage): aligned and ragged lengths, many tiles,
    fp32 and input-dtype accumulation, against the oracle on sampled rows."""
    tm, tn = tiles
    q, k, v = inputs((1, 2, s, 256), dtype, 2560 + s + (tm or 0))
    rows = sample_rows(s, 64)
    ref = oracle_f32(q, k, v, causal=causal, rows=rows)
    for accum in ("fp32", "fp16"):
        say(f"D=256 {dtype} (1,2,{s},256) causal={causal} tiles=({tm},{tn}) accum={accum}")
        out = run_gpu(q, k, v, causal=causal, tile_m=tm, tile_n=tn, accum_mode=accum)
        tol = TOL[dtype] if accum == "fp32" else LOWP_TOL[dtype]
        check_close(as_f32(out, rows), ref, dtype, tol=tol, what=f"D=256 accum={accum}")


def test_wide_head_dim_rejects_128_key_tiles(gpu):
    q, k, v = inputs((1, 1, 64, 160), "float16", 5)
    say("wide D=160 with TILE_N=128 -> ValueError before launch")
    with pytest.raises(ValueError, match="TILE_N=128"):
        run_gpu(q, k, v, causal=False, tile_m=64, tile_n=128)


def test_chunked_head_dim_knob_matches_unchunked(gpu):
    """TILEDATTN_CHUNKED_HEAD_DIMS=96 computes the same attention as the unchunked path."""
    q, k, v = inputs((1, 2, 256, 96), "bfloat16", 96)
    say("chunked knob bf16 (1,2,256,96)")
    a = run_gpu(q, k, v, causal=True, chunked_head_dims="96")
    b = run_gpu(q, k, v, causal=True)
    check_close(as_f32(a), oracle_f32(q, k, v, causal=True), "bfloat16", what="chunked 96")
    assert bool((a == b).all())


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("causal", [False, True])
def test_rising_logits_lazy_rescale(gpu, dtype, causal):
    """Key logits rising along S (0 to 116 log2 units over the sequence, q constant): each
    key slice's running max grows by about 14.5 log2 units a step, so P reaches ~2^14.5
    against a stale reference point before the lazy rescale (threshold 2^15) moves it, and
    moves it again a step later.  Checks that such P packs to the input dtype and the
    rescales keep O/l exact, against the oracle."""
    import torch

    s, d = 1024, 64
    q = torch.ones(1, 2, s, d, dtype=torch.float32)
    beta = torch.linspace(0.0, 116.0 / (8.0 * 1.4426950408889634), s)  # scale 1/8: s*c = 11.54 beta
    k = beta.view(1, 1, s, 1).expand(1, 2, s, d).clone()
    g = torch.Generator().manual_seed(7)
    v = torch.randn(1, 2, s, d, generator=g)
    q, k, v = (t.to(getattr(torch, dtype)) for t in (q, k, v))
    ref = oracle_f32(q, k, v, causal=causal)
    say(f"rising logits {dtype} (1,2,{s},{d}) causal={causal}")
    for tile in ((None, None), (128, 64), (64, 64)):
        out = run_gpu(q, k, v, causal=causal, tile_m=tile[0], tile_n=tile[1])
        check_close(as_f32(out), ref, dtype, what=f"rising logits tile={tile}")


def test_custom_scale(gpu):
    q, k, v = inputs((1, 4, 300, 64), "float16", 11)
    for scale in (0.05, 1.0, 0.3):
        say(f"scale={scale} fp16 (1,4,300,64)")
        out = run_gpu(q, k, v, causal=True, scale=scale)
        check_close(as_f32(out), oracle_f32(q, k, v, causal=True, scale=scale), "float16", what=f"scale {scale}")


# ---------------------------------------------------------------- accumulation in the input dtype

@pytest.mark.parametrize("dtype,d,causal", [("float16", 64, False), ("bfloat16", 128, True),
                                            ("float16", 128, True), ("bfloat16", 64, False)])
def test_input_dtype_accumulation(gpu, dtype, d, causal):
    """ACCUM_MODE=fp16: O kept in the input dtype between key tiles (flash_fwd.py:301-372)."""
    from oracle import oracle as O

    q, k, v = inputs((1, 4, 1000, d), dtype, 31)
    ref = oracle_f32(q, k, v, causal=causal)
    dc = O.dtype_code(dtype)
    for tm, tn in TILES:
        say(f"accum=input {dtype} (1,4,1000,{d}) causal={causal} tiles=({tm},{tn})")
        out = run_gpu(q, k, v, causal=causal, tile_m=tm, tile_n=tn, accum_mode="fp16")
        got = as_f32(out)
        check_close(got, ref, dtype, tol=LOWP_TOL[dtype], what=f"accum=input vs fp32 oracle tiles={tm},{tn}")
        emu = O.upcast(O.flash_tiled(O.to_bits(q), O.to_bits(k), O.to_bits(v), dc, causal=causal,
                                     tile_m=tm, tile_n=tn, accum_lowp=True), dc)
        check_close(got, emu, dtype, tol=TOL[dtype], what=f"accum=input vs tiled emulation tiles={tm},{tn}")


# ---------------------------------------------------------------- layout and launch plumbing

def test_strided_inputs_match_contiguous(gpu):
    """[B,S,H,D]-stored tensors viewed as [B,H,S,D] run without a copy and match."""
    import torch

    q, k, v = inputs((2, 4, 333, 128), "float16", 5)
    say("strided views fp16 (2,4,333,128)")
    qs, ks, vs = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v))
    assert not qs.is_contiguous()
    a = run_gpu(qs, ks, vs, causal=True)
    b = run_gpu(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert bool((a == b).all())
    check_close(as_f32(a), oracle_f32(q, k, v, causal=True), "float16", what="strided")


def test_non_default_stream_and_sync_modes(gpu):
    import torch

    from tiledattention import sdpa
    from tests.parity_util import knobs

    q, k, v = (t.cuda() for t in inputs((1, 2, 512, 64), "bfloat16", 9))
    ref = oracle_f32(q.cpu(), k.cpu(), v.cpu(), causal=False)
    s = torch.cuda.Stream()
    for mode in ("async", "post", "strict"):
        say(f"stream + sync_mode={mode}")
        with torch.cuda.stream(s), knobs(sync_mode=mode):
            out = sdpa(q, k, v)
        s.synchronize()
        check_close(as_f32(out), ref, "bfloat16", what=f"sync {mode}")


def test_zero_size_inputs(gpu):
    import torch

    from tiledattention import sdpa

    say("zero-size inputs")
    for shape in [(0, 2, 16, 64), (1, 0, 16, 64), (1, 2, 0, 64)]:
        q = torch.zeros(shape, dtype=torch.float16, device="cuda")
        out = sdpa(q, q, q, causal=True)
        assert out.shape == shape


def test_invalid_knobs_raise_before_launch(gpu):
    import torch

    from tiledattention import sdpa
    from tests.parity_util import knobs

    q = torch.zeros((1, 1, 64, 64), dtype=torch.float16, device="cuda")
    say("invalid knobs")
    for env, msg in [({"tile_m": 32}, "Unsupported tile"), ({"tile_n": "x"}, "must be an integer"),
                     ({"accum_mode": "fp8"}, "ACCUM_MODE"), ({"sync_mode": "later"}, "SYNC_MODE"),
                     ({"tile_m": -64}, "must be positive")]:
        with knobs(**env), pytest.raises(ValueError, match=msg):
            sdpa(q, q, q)
    with pytest.raises(Exception, match="head dimension D=300"):
        sdpa(*(torch.zeros((1, 1, 8, 300), dtype=torch.float16, device="cuda"),) * 3)


# ---------------------------------------------------------------- known-answer tests on the GPU

@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_kat_causal_row0_is_v0_exactly(gpu, dtype):
    q, k, v = inputs((2, 4, 700, 128), dtype, 3)
    say(f"KAT row0 {dtype}")
    out = run_gpu(q, k, v, causal=True)
    assert bool((out[:, :, 0, :].cpu() == v[:, :, 0, :]).all())


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_kat_constant_values(gpu, dtype):
    import torch

    q, k, _ = inputs((1, 3, 257, 64), dtype, 4)
    v = torch.full(q.shape, 0.75, dtype=q.dtype)
    for causal in (False, True):
        say(f"KAT constant v {dtype} causal={causal}")
        out = run_gpu(q, k, v, causal=causal)
        # P is rounded to the input dtype before P.V while l sums the unrounded P (as in
        # the reference), so the result is 0.75 up to that rounding, not bit-exact.
        check_close(as_f32(out), v.float().numpy(), dtype, what="constant v")


def test_kat_zero_keys_give_prefix_mean(gpu):
    import torch

    q, _, v = inputs((1, 2, 300, 64), "float16", 6)
    k = torch.zeros_like(q)
    vf = v.float()
    say("KAT k=0 prefix mean")
    out = run_gpu(q, k, v, causal=True)
    ref = (vf.cumsum(2) / torch.arange(1, 301).view(1, 1, -1, 1)).numpy()
    check_close(as_f32(out), ref, "float16", what="prefix mean")
    out = run_gpu(q, k, v, causal=False)
    check_close(as_f32(out), vf.mean(2, keepdim=True).expand_as(vf).numpy(), "float16", what="mean")


def test_kat_noncausal_key_permutation_invariance(gpu):
    import torch

    q, k, v = inputs((1, 2, 512, 128), "bfloat16", 8)
    perm = torch.randperm(512, generator=torch.Generator().manual_seed(1))
    say("KAT key permutation")
    a = as_f32(run_gpu(q, k, v, causal=False))
    b = as_f32(run_gpu(q, k[:, :, perm], v[:, :, perm], causal=False))
    check_close(a, b, "bfloat16", what="permuted keys")


def test_kat_heads_are_independent(gpu):
    q, k, v = inputs((2, 3, 200, 64), "float16", 12)
    say("KAT head independence")
    full = as_f32(run_gpu(q, k, v, causal=True))
    one = as_f32(run_gpu(q[1:2, 2:3], k[1:2, 2:3], v[1:2, 2:3], causal=True))
    assert np.array_equal(full[1:2, 2:3], one)


def test_golden_fixture_c1(gpu):
    """Committed golden vectors (tests/golden/c1.npz) through the GPU path."""
    from tests.golden.fixtures import load_fixture

    fx = load_fixture("c1")
    say("golden c1")
    out = run_gpu(fx["q"], fx["k"], fx["v"], causal=bool(fx["causal"]))
    check_close(as_f32(out), fx["out_f32"], str(fx["dtype"]), what="golden c1")


@pytest.mark.parametrize("shape,dtype,tiles", [
    ((4, 16, 2048, 128), "bfloat16", (128, 64)),
    ((8, 7, 2100, 64), "float16", (128, 64)),      # ragged: the tail-masked variant
    ((2, 28, 2304, 120), "bfloat16", (128, 128)),  # kernel head dim 128, columns 120.. zero
    ((8, 8, 2000, 128), "float16", (128, 64)),
    ((1, 8, 8192, 128), "bfloat16", (128, 64)),    # one block per CU
])
def test_rows256_noncausal(gpu, shape, dtype, tiles):
    """Non-causal grids whose 256-row blocks need at most half the rounds of 128-row ones
    run ta_fwd_pp256_* (the two wave groups on different rows, every key of a step each):
    sampled rows against the oracle, contiguous and [B,S,H,D] views."""
    import torch

    from tiledattention import sdpa
    from tiledattention.kernels import flash_fwd

    b, h, s, d = shape
    q, k, v = inputs(shape, dtype, 256 + s + d)
    rows = sample_rows(s, 64)
    ref = oracle_f32(q, k, v, causal=False, rows=rows)
    say(f"256-row blocks {dtype} {shape} non-causal tiles={tiles}")
    with knobs(tile_m=tiles[0], tile_n=tiles[1], accum_mode="fp32"):
        desc = flash_fwd.describe_call(q.to("cuda:0"), k.to("cuda:0"), v.to("cuda:0"), causal=False)
    assert desc["kernel"].startswith("ta_fwd_pp256_"), desc
    out = run_gpu(q, k, v, causal=False, tile_m=tiles[0], tile_n=tiles[1], accum_mode="fp32")
    check_close(as_f32(out, rows), ref, dtype, what=f"256-row {shape}")
    dev = torch.device("cuda:0")
    bshd = [t.transpose(1, 2).contiguous().to(dev).transpose(1, 2) for t in (q, k, v)]
    say(f"256-row blocks {dtype} {shape} non-causal [B,S,H,D] views")
    with knobs(tile_m=tiles[0], tile_n=tiles[1], accum_mode="fp32"):
        out = sdpa(*bshd, causal=False)
    torch.cuda.synchronize()
    check_close(as_f32(out, rows), ref, dtype, what=f"256-row {shape} BSHD")
