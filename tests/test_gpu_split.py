"""GPU parity of split key ranges (ta_sdpa_fwd_split: the split eight-wave kernel plus the
merge kernel) against the CPU oracle, and against the whole-row path on the same inputs.

Every case names itself on stdout before touching the GPU.  Chunk lengths are forced with
TILEDATTN_SPLIT so that every numbering shape runs: one-step chunks (every block split as
far as it goes), chunks that leave a remainder, non-causal and causal grids, ragged S
(masked last key step inside the last chunk), both dtypes and both head dims, strided
inputs, and the C5 outlier variant that stresses the rescale across chunk boundaries.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from tests.parity_util import as_f32, check_close, inputs, knobs, oracle_f32, run_gpu, sample_rows, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,dtype,causal,chunks", [
    ((1, 8, 1024, 128), "bfloat16", True, (1, 2, 3)),
    ((1, 2, 1000, 64), "float16", True, (1, 3)),
    ((2, 3, 777, 128), "float16", False, (1, 2, 5)),
    ((1, 8, 2048, 64), "bfloat16", False, (4,)),
    ((1, 4, 2304, 128), "float16", True, (5,)),
    ((1, 1, 129, 128), "bfloat16", True, (1,)),
    ((1, 1, 129, 64), "float16", False, (1,)),
    ((1, 4, 1300, 160), "bfloat16", True, (1, 3)),
    ((2, 2, 900, 160), "float16", False, (2,)),
    ((1, 3, 1000, 144), "bfloat16", True, (2,)),   # in-kernel padding to 160
])
def test_forced_chunks_match_oracle(gpu, shape, dtype, causal, chunks):
    q, k, v = inputs(shape, dtype, 300 + shape[2])
    ref = oracle_f32(q, k, v, causal=causal)
    for chunk in chunks:
        say(f"split {dtype} {shape} causal={causal} chunk={chunk}")
        # the automatic accumulation policy picks input-dtype accumulation for some of these
        # shapes, which has no split kernel
        out = run_gpu(q, k, v, causal=causal, split=chunk, accum_mode="fp32")
        check_close(as_f32(out), ref, dtype, what=f"split chunk={chunk}")


@pytest.mark.parametrize("shape,dtype,causal,chunks,tn", [
    ((1, 8, 2048, 128), "bfloat16", True, (1, 2, 4, 8), 64),   # C3 S=2048
    ((1, 8, 1024, 128), "bfloat16", True, (1, 3), 128),
    ((1, 8, 512, 128), "float16", True, (1, 2), 64),
    ((1, 2, 1000, 64), "float16", True, (1, 3), 64),           # ragged: the last half past S
    ((2, 3, 777, 128), "float16", False, (1, 2, 5), 64),
    ((1, 8, 1024, 64), "float16", False, (2, 4), 64),           # C2's shape
    ((1, 1, 129, 128), "bfloat16", True, (1,), 64),
    ((1, 4, 1300, 160), "bfloat16", True, (1, 3), 64),
    ((1, 3, 1000, 96), "float16", False, (2,), 128),
    ((1, 3, 700, 72), "bfloat16", True, (2,), 64),              # in-kernel padding to 96
    ((1, 2, 320, 144), "float16", True, (1,), 64),              # to 160; S = 5 blocks of 64 rows
])
def test_64_row_chunks_match_oracle(gpu, shape, dtype, causal, chunks, tn):
    """Split key ranges on the 64-row kernel (ta_fwd_pp64_split_*: each item of the 128-row
    numbering as two 64-row halves, the same merge kernel): forced chunk lengths against the
    oracle and against the 64-row whole-row kernel on the same inputs."""
    import torch

    from tests.parity_util import kernel_for

    q, k, v = inputs(shape, dtype, 640 + shape[2] + shape[3])
    ref = oracle_f32(q, k, v, causal=causal)
    say(f"64-row whole rows {dtype} {shape} causal={causal} tiles=(64,{tn})")
    whole = run_gpu(q, k, v, causal=causal, split="off", tile_m=64, tile_n=tn, accum_mode="fp32")
    check_close(as_f32(whole), ref, dtype, what="64-row whole rows")
    for chunk in chunks:
        kern = kernel_for(q, k, v, causal=causal, split=chunk, tile_m=64, tile_n=tn, accum_mode="fp32")
        say(f"64-row split {dtype} {shape} causal={causal} chunk={chunk} kernel={kern}")
        out = run_gpu(q, k, v, causal=causal, split=chunk, tile_m=64, tile_n=tn, accum_mode="fp32")
        check_close(as_f32(out), ref, dtype, what=f"64-row split chunk={chunk}")
        d = (out.float() - whole.float()).abs().max().item()
        assert d <= 2.0 ** -7 * max(1.0, float(whole.float().abs().max())), d
        assert torch.isfinite(out).all()


@pytest.mark.parametrize("shape", [(1, 8, 2048, 128), (1, 1, 8192, 128), (1, 2, 4096, 128), (1, 8, 2048, 160)])
def test_split_and_whole_rows_agree(gpu, shape):
    """bf16 causal, seed 1234, forced 8-step chunks (C3's shape) and the automatic plan
    (which splits the B*H = 1 and 2 shapes): both paths meet the oracle's tolerance and
    differ from each other only by the rounding of the merge."""
    from tiledattention.kernels import flash_fwd

    s, n_bh = shape[2], shape[1]
    q, k, v = inputs(shape, "bfloat16", 1234)
    rows = None if s <= 2048 else sample_rows(s, 128)
    ref = oracle_f32(q, k, v, causal=True, rows=rows)
    split = 8 if n_bh == 8 else "auto"
    say(f"bf16 causal {shape} split={split}")
    auto = run_gpu(q, k, v, causal=True, split=split)
    if n_bh < 8:
        assert any(key[0] == s and key[1] == n_bh and key[2] == 1 and c > 0
                   for key, c in flash_fwd._SPLIT_PLANS.items()), flash_fwd._SPLIT_PLANS
    say(f"bf16 causal {shape} split=off tiles=(128,64)")
    # the 128-row kernel's whole rows (the default tile for small grids is 64 rows)
    whole = run_gpu(q, k, v, causal=True, split="off", tile_m=128, tile_n=64)
    a, w = as_f32(auto, rows), as_f32(whole, rows)
    check_close(a, ref, "bfloat16", what=f"{shape} split {split}")
    check_close(w, ref, "bfloat16", what=f"{shape} whole rows")
    # one bf16 rounding step apart at most (|o| < 2 here, so 2^-7 per unit of |o|)
    diff = np.abs(a - w)
    assert float(diff.max()) <= 2.0 ** -7 * max(1.0, float(np.abs(w).max())), float(diff.max())
    assert float(diff.mean()) < 1e-3


def test_outlier_keys_across_chunks(gpu):
    """C5b's outlier variant (1% of k entries x20) at S=2048: the running maxima differ
    strongly between chunks, so the merge's log-sum-exp weights span many octaves."""
    q, k, v = inputs((1, 8, 2048, 128), "float16", 1234, outlier_frac=0.01, outlier_gain=20.0,
                     outlier_seed=1235)
    ref = oracle_f32(q, k, v, causal=True)
    for chunk in (1, 4):
        say(f"split fp16 outliers (1,8,2048,128) causal chunk={chunk}")
        out = run_gpu(q, k, v, causal=True, split=chunk, accum_mode="fp32")
        check_close(as_f32(out), ref, "float16", what=f"outliers chunk={chunk}")


def test_strided_inputs_and_scale(gpu):
    """[B,S,H,D]-strided views (no copy: unit last stride, 16-byte rows) and an explicit scale."""
    import torch

    from tiledattention import sdpa

    q, k, v = inputs((2, 4, 640, 64), "bfloat16", 77)
    ref = oracle_f32(q, k, v, causal=True, scale=0.3)
    dev = torch.device("cuda:0")
    qs, ks, vs = (t.transpose(1, 2).contiguous().to(dev).transpose(1, 2) for t in (q, k, v))
    assert not qs.is_contiguous()
    say("split bf16 strided (2,4,640,64) causal scale=0.3 chunk=2")
    with knobs(split=2, accum_mode="fp32"):
        out = sdpa(qs, ks, vs, causal=True, scale=0.3)
    torch.cuda.synchronize()
    check_close(as_f32(out), ref, "bfloat16", what="strided split")


def test_cabi_chunk_zero_is_the_whole_row_launch(gpu):
    """ta_sdpa_fwd_split with chunk 0 (or a chunk that splits nothing) is ta_sdpa_fwd: the
    outputs are bit-identical."""
    import torch

    from tiledattention import _lib

    lib = _lib.load()
    q, k, v = inputs((1, 2, 512, 128), "float16", 5)
    dev = torch.device("cuda:0")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    outs = [torch.full_like(qd, float("nan")) for _ in range(3)]

    def args(o):
        a = _lib.FwdArgs()
        a.q, a.k, a.v, a.o = qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), o.data_ptr()
        a.B, a.H, a.S, a.D = 1, 2, 512, 128
        for name, t in (("q_stride", qd), ("k_stride", kd), ("v_stride", vd), ("o_stride", o)):
            getattr(a, name)[:] = tuple(t.stride())
        a.scale, a.causal, a.dtype = 128 ** -0.5, 1, _lib.TA_FP16
        a.tile_m, a.tile_n, a.accum, a.device, a.sched = 128, 64, _lib.TA_ACC_FP32, 0, 1
        return a

    stream = torch.cuda.current_stream(dev).cuda_stream
    say("C-ABI fp16 (1,2,512,128) causal: ta_sdpa_fwd vs ta_sdpa_fwd_split chunk 0 and chunk 4")
    assert lib.ta_sdpa_fwd(ctypes.byref(args(outs[0])), ctypes.c_void_p(stream)) == _lib.TA_OK
    assert lib.ta_sdpa_fwd_split(ctypes.byref(args(outs[1])), 0, None, 0, ctypes.c_void_p(stream)) == _lib.TA_OK
    # 512 keys = 4 steps: a 4-step chunk splits nothing and needs no workspace
    assert lib.ta_sdpa_fwd_split(ctypes.byref(args(outs[2])), 4, None, 0, ctypes.c_void_p(stream)) == _lib.TA_OK
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    check_close(as_f32(outs[0]), oracle_f32(q, k, v, causal=True), "float16", what="C-ABI whole rows")


def test_cabi_split_with_caller_workspace(gpu):
    """The C ABI with a caller-owned workspace (torch allocation), reused by two calls of
    different shapes in a row on one stream; the workspace starts as garbage."""
    import torch

    from tiledattention import _lib

    lib = _lib.load()
    dev = torch.device("cuda:0")
    ws = torch.full((64 << 20,), 0x7f, dtype=torch.uint8, device=dev)  # NaN-ish bytes
    stream = torch.cuda.current_stream(dev).cuda_stream
    for shape, causal, chunk in (((1, 4, 1536, 128), 1, 2), ((1, 2, 700, 64), 0, 1),
                                 ((1, 2, 700, 160), 1, 2), ((1, 2, 2100, 96), 1, _lib.TA_SPLIT_PAIRS)):
        q, k, v = inputs(shape, "bfloat16", 11 + shape[2])
        qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
        o = torch.empty_like(qd)
        a = _lib.FwdArgs()
        a.q, a.k, a.v, a.o = qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), o.data_ptr()
        a.B, a.H, a.S, a.D = shape
        for name, t in (("q_stride", qd), ("k_stride", kd), ("v_stride", vd), ("o_stride", o)):
            getattr(a, name)[:] = tuple(t.stride())
        a.scale, a.causal, a.dtype = shape[3] ** -0.5, causal, _lib.TA_BF16
        a.tile_m, a.tile_n, a.accum, a.device, a.sched = 128, 64, _lib.TA_ACC_FP32, 0, 1
        need = ctypes.c_int64(0)
        assert lib.ta_split_workspace_size(ctypes.byref(a), chunk, ctypes.byref(need)) == _lib.TA_OK
        assert 0 < need.value <= ws.numel()
        say(f"C-ABI split bf16 {shape} causal={causal} chunk={chunk} workspace={need.value}")
        st = lib.ta_sdpa_fwd_split(ctypes.byref(a), chunk, ctypes.c_void_p(ws.data_ptr()), need.value,
                                   ctypes.c_void_p(stream))
        assert st == _lib.TA_OK, _lib.last_error(lib)
        torch.cuda.synchronize()
        check_close(as_f32(o), oracle_f32(q, k, v, causal=bool(causal)), "bfloat16",
                    what=f"C-ABI split {shape}")


@pytest.mark.parametrize("shape,dtype", [
    ((1, 8, 4096, 128), "bfloat16"),   # C3 S=4096: 16 pairs a head, 13 of them cut
    ((1, 2, 1000, 64), "float16"),     # ragged last block
    ((1, 3, 1300, 160), "bfloat16"),   # odd nq: the middle block alone
    ((2, 2, 2100, 96), "float16"),     # native D = 96, odd nq, ragged
    ((1, 4, 1000, 144), "bfloat16"),   # in-kernel padding to 160
    ((1, 1, 129, 128), "float16"),     # two blocks: no pair is cut, whole rows
])
def test_paired_split_matches_oracle(gpu, shape, dtype):
    """TILEDATTN_SPLIT=pairs (TA_SPLIT_PAIRS): causal blocks p and nq - 1 - p over two
    workgroups, the heavy block's key range cut between them and merged."""
    s = shape[2]
    q, k, v = inputs(shape, dtype, 500 + s)
    rows = None if s <= 2100 else sample_rows(s, 128)
    ref = oracle_f32(q, k, v, causal=True, rows=rows)
    say(f"paired split {dtype} {shape} causal")
    out = run_gpu(q, k, v, causal=True, split="pairs", accum_mode="fp32")
    check_close(as_f32(out, rows), ref, dtype, what=f"paired split {shape}")
    if s <= 2100:
        # block ids head by head instead of regrouped per XCD (TILEDATTN_SCHED=0)
        say(f"paired split {dtype} {shape} causal sched=0")
        out = run_gpu(q, k, v, causal=True, split="pairs", accum_mode="fp32", sched=0)
        check_close(as_f32(out, rows), ref, dtype, what=f"paired split {shape} sched 0")


def test_paired_split_outliers_and_whole_rows_agree(gpu):
    """C5b's fp16 outlier keys at S=4096 (running maxima differ strongly between the two
    chunks of a cut block): the paired split meets the oracle and stays within one fp16
    rounding of the whole-row result; a non-causal call with pairs is the whole-row
    launch."""
    import torch

    shape = (1, 8, 4096, 128)
    q, k, v = inputs(shape, "float16", 1234, outlier_frac=0.01, outlier_gain=20.0, outlier_seed=1235)
    rows = sample_rows(4096, 128)
    ref = oracle_f32(q, k, v, causal=True, rows=rows)
    say("paired split fp16 outliers (1,8,4096,128) causal")
    paired = run_gpu(q, k, v, causal=True, split="pairs", accum_mode="fp32")
    say("whole rows fp16 outliers (1,8,4096,128) causal")
    whole = run_gpu(q, k, v, causal=True, split="off", tile_m=128, tile_n=64, accum_mode="fp32")
    a, w = as_f32(paired, rows), as_f32(whole, rows)
    check_close(a, ref, "float16", what="paired split outliers")
    check_close(w, ref, "float16", what="whole rows outliers")
    # one fp16 rounding step apart at most (2^-10 per unit of |o|, twice for the margin)
    diff = np.abs(a - w)
    assert float(diff.max()) <= 2.0 ** -9 * max(1.0, float(np.abs(w).max())), float(diff.max())
    say("paired split bf16 (1,2,640,128) non-causal = whole rows")
    q, k, v = inputs((1, 2, 640, 128), "bfloat16", 9)
    p_nc = run_gpu(q, k, v, causal=False, split="pairs")
    w_nc = run_gpu(q, k, v, causal=False, split="off", tile_m=128, tile_n=64)
    assert torch.equal(p_nc, w_nc)


def test_automatic_plan_runs_the_paired_split(gpu):
    """B1 H6 S4096 bf16 causal: 192 query blocks of 128 rows for 256 CUs, 32 a head, so the
    library's plan (TILEDATTN_SPLIT unset) is the paired split; sampled rows meet the oracle."""
    from tiledattention import _lib
    from tiledattention.kernels import flash_fwd

    shape = (1, 6, 4096, 128)
    q, k, v = inputs(shape, "bfloat16", 4096)
    rows = sample_rows(4096, 96)
    ref = oracle_f32(q, k, v, causal=True, rows=rows)
    say("automatic plan bf16 (1,6,4096,128) causal")
    out = run_gpu(q, k, v, causal=True, split=None)
    assert any(key[0] == 4096 and key[1] == 6 and key[2] == 1 and c == _lib.TA_SPLIT_PAIRS
               for key, c in flash_fwd._SPLIT_PLANS.items()), flash_fwd._SPLIT_PLANS
    check_close(as_f32(out, rows), ref, "bfloat16", what="automatic paired split")


@pytest.mark.parametrize("shape,dtype,split,tm", [
    ((1, 8, 4096, 128), "bfloat16", "pairs", 128),   # paired split: 13 cut pairs a head
    ((2, 3, 777, 128), "float16", 4, 128),           # non-causal chunks of 4 steps (2 a block)
    ((1, 8, 2048, 128), "bfloat16", 4, 64),          # 64-row halves: 2 arrivals a chunk,
                                                     # 96 split blocks of up to 4 chunks
])
def test_in_kernel_merge_repeated_and_on_many_streams(gpu, shape, dtype, split, tm):
    """Split launches are merged by their own last workgroup per block (arrival counters
    per (device, stream), left at zero by every launch).  Forty back-to-back calls on one
    stream give bit-identical outputs (a counter not reset would merge early or never);
    the same call on 20 streams, more than the 16 counter regions, so the last streams
    run the merge kernel instead, gives the same bits everywhere; and it meets the oracle."""
    import torch

    from tiledattention import sdpa
    from tiledattention.kernels import flash_fwd

    causal = split == "pairs" or shape[2] != 777
    s = shape[2]
    q, k, v = inputs(shape, dtype, 700 + s)
    rows = None if s <= 2048 else sample_rows(s, 96)
    ref = oracle_f32(q, k, v, causal=causal, rows=rows)
    dev = torch.device("cuda:0")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    kn = dict(split=split, tile_m=tm, tile_n=64, accum_mode="fp32")
    with knobs(**kn):
        desc = flash_fwd.describe_call(qd, kd, vd, causal=causal)
    assert desc["merge_kernel"] and desc["merge_in_kernel"] == 1, desc
    say(f"in-kernel merge {dtype} {shape} split={split} rows={tm}: 40 calls on one stream")
    with knobs(**kn):
        first = sdpa(qd, kd, vd, causal=causal)
        outs = [sdpa(qd, kd, vd, causal=causal) for _ in range(40)]
    torch.cuda.synchronize()
    assert all(torch.equal(o, first) for o in outs)
    check_close(as_f32(first, rows), ref, dtype, what=f"in-kernel merge {shape}")
    say(f"in-kernel merge {dtype} {shape} split={split} rows={tm}: 20 streams")
    streams = [torch.cuda.Stream(dev) for _ in range(20)]
    per = []
    with knobs(**kn):
        for st in streams:
            st.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(st):
                per.append(sdpa(qd, kd, vd, causal=causal))
    torch.cuda.synchronize()
    for i, o in enumerate(per):
        assert torch.equal(o, first), f"stream {i}: max |diff| {float((o.float() - first.float()).abs().max())}"


def test_split_launch_in_a_hip_graph(gpu):
    """A split launch merged in the kernel (the paired split at C3's S=4096 shape, on fewer
    heads) captured in a HIP graph (torch.cuda.graph) and replayed five times, with eager
    work and synchronisations between the replays: every replay equals the eager result
    (the arrival counters are left at zero by every launch, so a replay needs no reset), and
    the eager result meets the oracle.  The code object is loaded by an eager call first."""
    import torch

    from tiledattention import sdpa
    from tiledattention.kernels import flash_fwd

    shape = (1, 2, 4096, 128)
    q, k, v = inputs(shape, "bfloat16", 4242)
    rows = sample_rows(4096, 96)
    ref = oracle_f32(q, k, v, causal=True, rows=rows)
    dev = torch.device("cuda:0")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    with knobs(split="pairs", tile_m=128, tile_n=64, accum_mode="fp32"):
        desc = flash_fwd.describe_call(qd, kd, vd, causal=True)
        assert desc["layout"] == 4 and desc["merge_in_kernel"] == 1, desc
        say("split launch in a HIP graph: eager call")
        eager = sdpa(qd, kd, vd, causal=True)
        torch.cuda.synchronize()
        s = torch.cuda.Stream(dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s):
            sdpa(qd, kd, vd, causal=True)  # warm the plan cache on the capture stream
        torch.cuda.current_stream(dev).wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        say("split launch in a HIP graph: capture")
        with torch.cuda.graph(g):
            captured = sdpa(qd, kd, vd, causal=True)
    torch.cuda.synchronize()
    for i in range(5):
        say(f"split launch in a HIP graph: replay {i}")
        captured.fill_(float("nan"))
        g.replay()
        # eager work between replays, on the default stream
        _ = (qd.float() * 2).sum()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"replay {i}: max |diff| {float((captured.float() - eager.float()).abs().max())}"
    check_close(as_f32(eager, rows), ref, "bfloat16", what="split in a graph (eager)")
