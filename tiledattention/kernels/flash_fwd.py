"""Host side of the SDPA forward: knob policy, argument preparation, launch.

Keeps the reference's function names and policies (src/tiledattention/kernels/
flash_fwd.py:12-259, 786-973) so that callers and tests written against it read the same,
and replaces its cuTile launch with one call into the C ABI (``ta_sdpa_fwd``) on torch's
current HIP stream of the inputs' device.

Environment knobs are re-read on every call, as in the reference:

``TILEDATTN_TILE_M`` / ``TILEDATTN_TILE_N``
    Query rows per workgroup / keys per tile.  If either is set, the other defaults to 64
    (flash_fwd.py:68-84, 851-856); non-integers and non-positive values raise
    ``ValueError`` as there.  The gfx950 kernels exist for 64 and 128 only; any other
    positive value raises ``ValueError`` naming the supported set.  When neither is set
    the tile is chosen by ``_default_tile_config_for_shape_gfx950``.
``TILEDATTN_ACCUM_MODE``
    ``auto`` | ``fp32`` | ``fp16``; "fp16" accumulates in the input dtype (bf16 for bf16
    inputs).  Parsing restated from flash_fwd.py:123-146; ``auto`` resolves to fp32 on
    gfx950 (``_default_accum_mode_for_shape_gfx950``), where the reference's shape rule
    (flash_fwd.py:102-120) would pick the slower input-dtype path.
``TILEDATTN_SYNC_MODE``
    ``async`` (default) | ``post`` | ``strict`` (flash_fwd.py:805-818).  Validated before
    the launch here (the reference validates after launching).
``TILEDATTN_DISABLE_ALIGNED_FASTPATH``
    Parsed as flash_fwd.py:225-226 (anything but unset, "", "0", "false", "False"
    disables).  The fast path is the kernel variant without tail masking
    (``ta_fwd_args.aligned``): it runs when S is a multiple of both tile sizes, causal or
    not, unless this knob is set, which forces the tail-masked variant.  The reference's
    other conditions (non-causal, S >= 1024 / 2048, D in {64, 128}, flash_fwd.py:199-238)
    exist because its aligned kernel has no causal mask and was tuned on GB10; both
    variants compute the same result.
``TILEDATTN_KERNEL_OPT_LEVEL`` / ``_OCCUPANCY`` / ``_NUM_CTAS``
    Parsed as in flash_fwd.py:87-99 (``ValueError`` on non-integers) and kept in the cache
    key; the code objects are precompiled at -O3, so they do not change the kernel.
``TILEDATTN_CHUNKED_HEAD_DIMS``
    Parsed as in flash_fwd.py:166-196.  A chunked plan computes the same attention as the
    unchunked one, so here it runs the kernel that serves the head dim unchunked (96 on the
    native D = 96 kernel with 128-row tiles and fp32 accumulation, else on the D = 128
    kernel with in-kernel padding; 160 on the native D = 160 kernel).
``TILEDATTN_SCHED`` (this build only)
    Workgroup-to-tile order: ``0`` plain, ``1`` XCD-grouped (large causal grids on the
    eight-wave kernel run query blocks in pairs, see ``ta_fwd_args.sched``), ``2``
    XCD-grouped with causal heavy/light complementary order, ``3`` pairs whatever the grid
    size; default: see ``_resolve_sched``.
``TILEDATTN_SPLIT`` (this build only)
    Split key ranges (``ta_sdpa_fwd_split``): ``auto`` (default) asks the library's
    dispatch model (``ta_split_plan``), ``0``/``off`` never splits, a positive integer
    forces chunks of that many 128-key steps, ``pairs`` the paired split
    (``TA_SPLIT_PAIRS``: causal blocks p and nq - 1 - p balanced over two workgroups;
    non-causal calls run whole rows).  Splitting exists for tiles (128, 64) and (128, 128)
    with fp32 accumulation and kernel head dims up to 160; forcing it elsewhere raises
    ``ValueError``.
"""

from __future__ import annotations

import ctypes
import os
from typing import Any

from .. import _lib, _runtime
from .._errors import DTypeNotSupportedError, InvalidShapeError, TiledAttentionError
from . import compile_cache as _compile_cache
from .compile_cache import get_kernel

_DEFAULT_TM = 64
_DEFAULT_TN = 64
_CHUNKED_HEAD_DIM_PARTS = {
    96: (64, 32),
    160: (128, 32),
}
_SUPPORTED_TILES = frozenset({64, 128})
_KERNEL_HEAD_DIMS = (64, 128, 160, 256)
_WIDE_HEAD_DIM_TILE_N = 64  # head dims above 128 run with 64-key tiles only
_SYNC_MODES = ("strict", "post", "async")


def _dtype_code_for_torch_dtype(torch_dtype: Any) -> int:
    """fp16 -> TA_FP16, bf16 -> TA_BF16, else ``DTypeNotSupportedError`` (cf. flash_fwd.py:27-44)."""
    torch_mod = _runtime.get_torch_module()
    if torch_dtype == torch_mod.float16:
        return _lib.TA_FP16
    if torch_dtype == torch_mod.bfloat16:
        return _lib.TA_BF16
    raise DTypeNotSupportedError("q dtype must be torch.float16 or torch.bfloat16.")


def _get_env_int(name: str, default: int | None) -> int | None:
    """Integer env knob; unset or blank -> ``default`` (flash_fwd.py:47-65)."""
    raw = os.getenv(name)
    if raw is None or raw.strip() == "":
        return default
    try:
        return int(raw)
    except ValueError as exc:
        raise ValueError(f"Environment variable {name} must be an integer.") from exc


def _resolve_tile_config() -> tuple[int, int]:
    """(TILE_M, TILE_N) from the environment; unset one defaults to 64 (flash_fwd.py:68-84)."""
    tile_m = _get_env_int("TILEDATTN_TILE_M", None)
    tile_n = _get_env_int("TILEDATTN_TILE_N", None)
    if tile_m is None:
        tile_m = _DEFAULT_TM
    if tile_n is None:
        tile_n = _DEFAULT_TN
    if tile_m <= 0 or tile_n <= 0:
        raise ValueError("TILEDATTN_TILE_M and TILEDATTN_TILE_N must be positive.")
    return tile_m, tile_n


def _check_tile_supported(tile_m: int, tile_n: int) -> None:
    if tile_m not in _SUPPORTED_TILES or tile_n not in _SUPPORTED_TILES:
        raise ValueError(
            f"Unsupported tile ({tile_m}, {tile_n}): the gfx950 kernels are built for "
            "TILEDATTN_TILE_M and TILEDATTN_TILE_N in {64, 128}."
        )


def _resolve_kernel_options() -> tuple[int, int | None, int | None]:
    """(opt_level, occupancy, num_ctas) as flash_fwd.py:87-99 parses them."""
    opt_level = _get_env_int("TILEDATTN_KERNEL_OPT_LEVEL", 3)
    occupancy = _get_env_int("TILEDATTN_KERNEL_OCCUPANCY", None)
    num_ctas = _get_env_int("TILEDATTN_KERNEL_NUM_CTAS", None)
    assert opt_level is not None
    return opt_level, occupancy, num_ctas


def _default_accum_mode_for_shape_gfx950(*, seq_len: int, head_dim: int, causal: bool) -> str:
    """``auto`` on gfx950: fp32 for every shape.  Input-dtype accumulation runs the four-wave
    kernels and rounds O after every key tile; fp32 runs the eight-wave kernel at the
    default tile.  On the MI355X, fp32 is 1.4-2.2x faster over the shapes where the
    reference's rule picks the input dtype (non-causal D = 64, S = 1024-16384, fp16 and
    bf16) and closer to the exact result."""
    del seq_len, head_dim, causal
    return "fp32"


def _resolve_accum_mode(*, seq_len: int, head_dim: int, causal: bool) -> str:
    """``TILEDATTN_ACCUM_MODE`` (auto|fp32|fp16, case-insensitive) -> 'fp32' | 'fp16' (flash_fwd.py:123-146)."""
    raw_mode = os.getenv("TILEDATTN_ACCUM_MODE")
    if raw_mode is None or raw_mode.strip() == "":
        return _default_accum_mode_for_shape_gfx950(seq_len=seq_len, head_dim=head_dim, causal=causal)
    mode = raw_mode.strip().lower()
    if mode == "auto":
        return _default_accum_mode_for_shape_gfx950(seq_len=seq_len, head_dim=head_dim, causal=causal)
    if mode not in {"fp32", "fp16"}:
        raise ValueError(
            f"Unsupported TILEDATTN_ACCUM_MODE={mode!r}. Use one of: auto, fp32, fp16."
        )
    return mode


def _resolve_kernel_head_dim_gfx950(head_dim: int, *, native_96: bool = False) -> tuple[int, int]:
    """Head dim of the gfx950 kernel that runs ``head_dim``, and the zero padding to add.

    Kernels exist for D = 64, 128, 160 and 256, and D = 96 on the eight-wave kernels with
    fp32 accumulation (``native_96``).  Other head
    dims are zero-padded to the next of them, which leaves Q K^T unchanged and only adds
    zero output columns that are sliced off (the reference pads the same way, to a power of
    two, flash_fwd.py:149-163; its 96 = 64 + 32 and 160 = 128 + 32 chunk plans, :21-24,
    compute the same contractions as the native D = 96 and 160 kernels here).  Above 256
    there is no kernel.
    """
    if head_dim <= 0:
        raise InvalidShapeError("head dimension D must be positive.")
    if native_96 and 64 < head_dim <= 96:
        return 96, 96 - head_dim
    for kd in _KERNEL_HEAD_DIMS:
        if head_dim <= kd:
            return kd, kd - head_dim
    raise InvalidShapeError(
        f"head dimension D={head_dim} is not supported: the gfx950 kernels cover D <= 256."
    )


def _resolve_chunk_plan(head_dim: int) -> tuple[tuple[int, int], ...] | None:
    """``TILEDATTN_CHUNKED_HEAD_DIMS`` plan for ``head_dim`` (flash_fwd.py:166-196)."""
    enabled = os.getenv("TILEDATTN_CHUNKED_HEAD_DIMS", "").strip()
    if enabled == "":
        return None
    try:
        enabled_dims = {int(x.strip()) for x in enabled.split(",") if x.strip() != ""}
    except ValueError as exc:
        raise ValueError(
            "Environment variable TILEDATTN_CHUNKED_HEAD_DIMS must be a comma-separated list of integers."
        ) from exc
    if head_dim not in enabled_dims:
        return None
    parts = _CHUNKED_HEAD_DIM_PARTS.get(head_dim)
    if parts is None:
        return None
    offset = 0
    plan: list[tuple[int, int]] = []
    for width in parts:
        plan.append((offset, width))
        offset += width
    return tuple(plan)


def _aligned_fastpath_disabled() -> bool:
    """``TILEDATTN_DISABLE_ALIGNED_FASTPATH`` as flash_fwd.py:225-226 reads it: any value
    other than unset, "", "0", "false" or "False" disables the fast path."""
    return os.getenv("TILEDATTN_DISABLE_ALIGNED_FASTPATH", "").strip() not in {"", "0", "false", "False"}


def _use_unmasked_tail_kernel(*, seq_len: int, tile_m: int, tile_n: int) -> bool:
    """The aligned fast path on gfx950: the kernel variant without tail masking, taken when
    every tile is whole (S a multiple of both tile sizes) unless the knob disables it.  The
    reference's predicate (flash_fwd.py:199-238) also requires non-causal, D in {64, 128},
    S >= 1024 (D = 64) / 2048 (D = 128) and no padding or chunk plan: its unmasked kernel has
    no causal mask and the thresholds are its GB10 tuning.  Here causal masking is separate
    from tail masking, and the two variants give the same result on such S."""
    if _aligned_fastpath_disabled():
        return False
    return seq_len % tile_m == 0 and seq_len % tile_n == 0


def _default_tile_config_for_shape_gfx950(*, seq_len: int, head_dim: int, causal: bool,
                                         n_bh: int = 0, accum_mode: str = "fp32",
                                         compute_units: int) -> tuple[int, int]:
    """Default (TILE_M, TILE_N) on gfx950 when neither env knob is set.

    128 query rows per workgroup: the eight-wave kernel (two waves per SIMD splitting every
    128-key step, one workgroup per CU; at kernel head dims above 128 with input-dtype
    accumulation the four-wave kernel with 64-key tiles).  When the 64-row blocks of all
    ``n_bh`` heads fit the CUs in one wave (B*H*ceil(S/64) <= CUs; head dims up to 128, or up
    to 160 with fp32 accumulation; ``compute_units`` is the device's CU count), 64 rows instead: the 64-row eight-wave kernel halves each
    block's key loop and the grid is still one workgroup per CU (B1 H8 bf16: causal S=1024
    15.0 -> 12.0 us, S=2048 23.5 -> 18.8; non-causal S=1024 14.4 -> 11.9, S=2048 23.3 ->
    20.3; D=64 causal S=2048 18.2 -> 13.5; D=160 S=512 / 1024 / 2048 causal 12.2 -> 10.0 /
    17.5 -> 13.1 / 28.3 -> 21.9, non-causal 12.3 -> 9.7 / 17.6 -> 13.0 / 28.3 -> 26.8).
    With more blocks than CUs, the second block of a CU pays the
    fixed cost of a workgroup again (B2 H16 S1024 causal: 16.4 -> 21.4 us), so 128 rows.
    The caller keeps 128 rows where the 128-row kernel would split key ranges
    (``_split_preferred``).

    TILE_N follows the reference's rule (flash_fwd.py:254-259): 128 for non-causal
    D = 128 at S >= 2048, else 64.  With fp32 accumulation both run the same kernels; with
    input-dtype accumulation it is the rounding cadence of O (once per TILE_N keys), so
    the default rounds as often as the reference's default does (C4 D = 128 bf16: 860 ->
    979 TFLOP/s against TILE_N = 64).
    """
    tile_n = 128 if (not causal and head_dim == 128 and seq_len >= 2048) else 64
    max_d64 = 160 if accum_mode == "fp32" else 128  # 64-row eight-wave kernels
    if (0 < head_dim <= max_d64 and n_bh > 0 and seq_len > 0
            and n_bh * ((seq_len + 63) // 64) <= compute_units):
        return 64, tile_n
    return 128, tile_n


def _resolve_sync_mode() -> str:
    """``TILEDATTN_SYNC_MODE`` -> 'async' | 'post' | 'strict' (flash_fwd.py:805-818), checked up front."""
    sync_mode = os.getenv("TILEDATTN_SYNC_MODE", "async").strip().lower()
    if sync_mode not in _SYNC_MODES:
        raise ValueError(
            f"Unsupported TILEDATTN_SYNC_MODE={sync_mode!r}. Use one of: strict, post, async."
        )
    return sync_mode


_CU_COUNTS: dict[int, int] = {}


def _compute_units(torch_mod, device_index: int) -> int:
    """The device's compute units (multiProcessorCount), read once per device."""
    n = _CU_COUNTS.get(device_index)
    if n is None:
        n = _CU_COUNTS[device_index] = int(torch_mod.cuda.get_device_properties(device_index).multi_processor_count)
    return n


def _workgroups_per_cu(*, tile_m: int, tile_n: int, accum_code: int, head_dim: int = 128,
                       causal: bool = True) -> int:
    """Workgroups of one launch resident on a CU at once: two for the non-causal eight-wave
    kernels at kernel head dim 64 with fp32 accumulation (built for 128 VGPRs, 64 KiB of
    LDS), one for the other eight-wave kernels (their stages fill a CU's LDS, or their
    registers two waves per SIMD); for the four-wave kernels two at 128x64 (input-dtype
    accumulation), two at 64x128 (one LDS stage), four at 64x64 up to D = 128 and two above
    (one LDS stage), one otherwise (LDS or registers)."""
    if _eight_wave_kernel(tile_m=tile_m, tile_n=tile_n, accum_code=accum_code,
                          kernel_head_dim=head_dim):
        fp32 = accum_code == _lib.TA_ACC_FP32
        return 2 if fp32 and head_dim <= 64 and not causal else 1
    if (tile_m, tile_n) == (128, 64) and accum_code == _lib.TA_ACC_INPUT:
        return 2
    if (tile_m, tile_n) == (64, 128) and head_dim <= 128:
        return 2  # one LDS stage (76 KiB at D = 128), one wave per SIMD
    if (tile_m, tile_n) == (64, 64):
        return 4 if head_dim <= 128 else 2  # one LDS stage; two waves per SIMD up to D = 128
    return 1


def _resolve_sched(*, n_blocks: int, causal: bool, tile_m: int, tile_n: int,
                   accum_code: int = _lib.TA_ACC_FP32, head_dim: int = 128,
                   compute_units: int) -> int:
    """Workgroup order.  XCD grouping needs the grid to split evenly over the 8 XCDs.  Causal
    tiles go heaviest first (each CU takes the next tile as its last one ends, pairing heavy
    with light ones); when every workgroup is resident at once on the device's
    ``compute_units`` CUs there is no "next", and the complementary order (sched 2) places
    heavy and light tiles on the same CU instead."""
    raw = os.getenv("TILEDATTN_SCHED", "").strip()
    if raw == "":
        if n_blocks % 8 != 0:
            return 0
        resident = compute_units * _workgroups_per_cu(tile_m=tile_m, tile_n=tile_n, accum_code=accum_code,
                                                  head_dim=head_dim, causal=causal)
        return 2 if causal and n_blocks <= resident else 1
    if raw not in {"0", "1", "2", "3"}:
        raise ValueError(f"Unsupported TILEDATTN_SCHED={raw!r}. Use 0, 1, 2 or 3.")
    return int(raw)


class _Launcher:
    """A kernel resolved in the native cache for one device; calling it enqueues a launch."""

    __slots__ = ("lib", "device", "config")

    def __init__(self, lib, device: int, config: tuple[int, ...]):
        self.lib = lib
        self.device = device
        self.config = config
        dtype, head_dim, tile_m, tile_n, causal, accum, aligned = config
        st = lib.ta_prepare(device, dtype, head_dim, tile_m, tile_n, causal, accum, aligned)
        _raise_for_status(lib, st)

    def __call__(self, args: _lib.FwdArgs, stream: int) -> None:
        st = self.lib.ta_sdpa_fwd(ctypes.byref(args), stream)  # c_void_p argtype takes the int
        if st:
            _raise_for_status(self.lib, st)

    def split(self, args: _lib.FwdArgs, chunk_steps: int, workspace: int, workspace_bytes: int,
              stream: int) -> None:
        st = self.lib.ta_sdpa_fwd_split(ctypes.byref(args), chunk_steps, ctypes.c_void_p(workspace),
                                        workspace_bytes, ctypes.c_void_p(stream))
        _raise_for_status(self.lib, st)


# (S, B*H, causal, device) -> chunk steps chosen by the library's dispatch model.
_SPLIT_PLANS: dict[tuple[int, int, int, int], int] = {}


_FAMILY: dict[tuple[int, int, int, int], tuple[bool, bool]] = {}


def _kernel_family(*, tile_m: int, tile_n: int, accum_code: int, kernel_head_dim: int) -> tuple[bool, bool]:
    """(eight-wave kernel, split kernels exist) for a configuration, as the library reports
    them (``ta_describe_launch_model``: ``in_place_pad``, ``split_capable``); (False, False)
    for a configuration the library has no kernel for."""
    key = (tile_m, tile_n, accum_code, kernel_head_dim)
    fam = _FAMILY.get(key)
    if fam is None:
        lib = _lib.load()
        args = _lib.shape_args(D=kernel_head_dim, tile_m=tile_m, tile_n=tile_n, accum=accum_code)
        out = _lib.LaunchDesc()
        st = lib.ta_describe_launch_model(ctypes.byref(args), 0, 256, ctypes.byref(out))
        fam = _FAMILY[key] = (bool(out.in_place_pad), bool(out.split_capable)) if st == _lib.TA_OK \
            else (False, False)
    return fam


def _eight_wave_kernel(*, tile_m: int, tile_n: int, accum_code: int, kernel_head_dim: int) -> bool:
    """Whether the configuration runs an eight-wave kernel, the ones with in-place padding of
    narrower head dims (fp32 accumulation with 128-row tiles at kernel head dims up to 160 or
    64-row tiles at 64, 96, 128 and 160; input-dtype accumulation with any tile at 64 or
    128).  Read from the library, whose kernel selection it is."""
    return _kernel_family(tile_m=tile_m, tile_n=tile_n, accum_code=accum_code,
                          kernel_head_dim=kernel_head_dim)[0]


def _split_capable(*, tile_m: int, tile_n: int, accum_code: int, kernel_head_dim: int) -> bool:
    """Whether split key ranges exist (the eight-wave kernels with fp32 accumulation: chunks
    and the paired split at 128 rows, chunks at 64 rows), as the library reports it."""
    return _kernel_family(tile_m=tile_m, tile_n=tile_n, accum_code=accum_code,
                          kernel_head_dim=kernel_head_dim)[1]


def _resolve_split(lib, args: _lib.FwdArgs, *, capable: bool, compute_units: int = 0) -> int:
    """``TILEDATTN_SPLIT`` -> chunk length in 128-key steps (0 = whole rows,
    ``_lib.TA_SPLIT_PAIRS`` = the paired split).  ``auto`` asks the library's dispatch
    model for a device of ``compute_units`` CUs (``ta_split_plan_model``), or for the
    arguments' device when 0 (``ta_split_plan``)."""
    raw = os.getenv("TILEDATTN_SPLIT", "").strip().lower()
    rows128 = int(args.tile_m) == 128
    if raw in ("", "auto"):
        if not capable:
            return 0
        key = (int(args.S), int(args.B * args.H), int(args.causal), int(compute_units) or -1 - int(args.device),
               int(args.tile_m), int(args.D))
        chunk = _SPLIT_PLANS.get(key)
        if chunk is None:
            if compute_units:
                chunk = int(lib.ta_split_plan_model_rows(int(args.S), int(args.B * args.H), int(args.causal),
                                                         int(args.D), int(args.tile_m), int(compute_units)))
            else:
                out = ctypes.c_int32(0)
                _raise_for_status(lib, lib.ta_split_plan(ctypes.byref(args), ctypes.byref(out)))
                chunk = int(out.value)
            _SPLIT_PLANS[key] = chunk
        return chunk
    if raw in ("0", "off"):
        return 0
    if raw == "pairs":
        if not capable or not rows128:
            raise ValueError(
                "TILEDATTN_SPLIT needs fp32 accumulation with tile (128, 64) or (128, 128) and a head "
                "dim of at most 160 (pairs: 128-row tiles only; chunks also on tile (64, 64) or "
                "(64, 128) with D = 64, 96, 128 or 160)."
            )
        return _lib.TA_SPLIT_PAIRS
    try:
        chunk = int(raw)
    except ValueError as exc:
        raise ValueError(
            f"TILEDATTN_SPLIT must be 'auto', 'off', 'pairs' or an integer, got {raw!r}.") from exc
    if chunk < 0:
        raise ValueError(f"TILEDATTN_SPLIT must be >= 0, got {chunk}.")
    if chunk and not capable:
        raise ValueError(
            "TILEDATTN_SPLIT needs fp32 accumulation with tile (128, 64) or (128, 128) and a head "
            "dim of at most 160 (pairs: 128-row tiles only; chunks also on tile (64, 64) or "
            "(64, 128) with D = 64, 96, 128 or 160)."
        )
    return chunk


def _split_preferred(lib, batch: int, heads: int, seq_len: int, head_dim: int, causal: bool,
                     compute_units: int, accum_mode: str = "fp32") -> bool:
    """Whether the 128-row kernel runs split key ranges for this shape (a forced chunk
    length, or the library's dispatch model under ``TILEDATTN_SPLIT=auto``): the default
    tile then stays at 128 rows, the tile the split path exists for.  Split kernels exist
    for fp32 accumulation only, so input-dtype accumulation never prefers them (128 rows
    would then run unsplit on half the CUs the 64-row default fills)."""
    if accum_mode != "fp32":
        return False
    raw = os.getenv("TILEDATTN_SPLIT", "").strip().lower()
    if raw in ("0", "off"):
        return False
    if raw not in ("", "auto"):
        return True
    kernel_head_dim, _ = _resolve_kernel_head_dim_gfx950(head_dim, native_96=True)
    args = _lib.shape_args(B=batch, H=heads, S=seq_len, D=kernel_head_dim, causal=causal)
    return _resolve_split(lib, args, capable=True, compute_units=compute_units) != 0


def _raise_for_status(lib, status: int) -> None:
    if status == _lib.TA_OK:
        return
    msg = f"{_lib.status_name(lib, status)}: {_lib.last_error(lib)}"
    if status == _lib.TA_EINVAL:
        raise InvalidShapeError(msg)
    if status == _lib.TA_EUNSUPPORTED:
        raise InvalidShapeError(msg)
    if status == _lib.TA_ENOKERNEL:
        from .._errors import DependencyError

        raise DependencyError(msg)
    raise TiledAttentionError(msg)


def _kernel_ready(torch_mod, t, width: int, pad_dim: int):
    """Tensor in a layout the kernel reads directly: [B,H,S,width] (width = the kernel's
    head dim, or the tensor's own when the kernel pads in place), unit last stride, 16-byte
    rows at a 16-byte aligned address (a fresh dense copy otherwise)."""
    if pad_dim > 0:
        return torch_mod.nn.functional.pad(t, (0, pad_dim)).contiguous()
    if _strides_ok(t.stride(), t.shape, width) and t.data_ptr() % 16 == 0:
        return t
    # contiguous() returns a dense but misaligned view unchanged; a clone is a new block
    return t.clone(memory_format=torch_mod.contiguous_format)


# The kernels address a (b, h) slice, and the 128 rows of one tile step, with 32-bit buffer
# offsets: a row stride below 2^23 elements keeps 128 rows below 2^31 bytes, and a slice
# must stay below 2^31 bytes (the same bounds the C ABI enforces).
_ROW_STRIDE_LIMIT = 1 << 23
_SLICE_BYTES_LIMIT = 1 << 31


def _strides_ok(stride, shape, width: int) -> bool:
    """Whether the kernels can read a [B, H, S, D] view with these element strides in place:
    unit last stride; the others non-negative multiples of 8 (16-byte rows); rows that do
    not overlap (row stride at least the width read; a zero row stride, as ``expand`` along
    S gives, would make a slice's buffer range empty and read zeros); and the 32-bit buffer
    ranges above.  Anything else is copied to a dense tensor first, as the reference copies
    every input (flash_fwd.py:865-867)."""
    seq_len, head_dim = int(shape[2]), int(shape[3])
    row = int(stride[2])
    return (stride[3] == 1 and all(x >= 0 and x % 8 == 0 for x in stride[:3]) and head_dim == width
            and width <= row < _ROW_STRIDE_LIMIT and seq_len * row * 2 < _SLICE_BYTES_LIMIT)


# Knobs this module reads, re-read on every call as in the reference.  A launch plan is
# cached per (shapes, strides, dtype, device, causal, knob values), so a changed knob
# builds a new plan exactly where the reference would change its behaviour.
_KNOBS = (
    "TILEDATTN_TILE_M", "TILEDATTN_TILE_N", "TILEDATTN_ACCUM_MODE", "TILEDATTN_SYNC_MODE",
    "TILEDATTN_DISABLE_ALIGNED_FASTPATH", "TILEDATTN_KERNEL_OPT_LEVEL",
    "TILEDATTN_KERNEL_OCCUPANCY", "TILEDATTN_KERNEL_NUM_CTAS", "TILEDATTN_CHUNKED_HEAD_DIMS",
    "TILEDATTN_SCHED", "TILEDATTN_SPLIT",
)
# os.environ keeps its encoded mapping in ``_data`` (CPython, POSIX); reading it directly
# skips the per-key encode/decode of os.getenv.  Assignments through os.environ (and
# os.putenv-free tools such as pytest's monkeypatch) update it.
_ENV_DATA = getattr(os.environ, "_data", None)
_KNOB_KEYS = tuple(os.environ.encodekey(n) for n in _KNOBS) if hasattr(os.environ, "encodekey") else None


def _knob_snapshot() -> tuple:
    if _ENV_DATA is not None and _KNOB_KEYS is not None:
        return tuple(map(_ENV_DATA.get, _KNOB_KEYS))
    return tuple(map(os.environ.get, _KNOBS))


class _LaunchPlan:
    """Everything a launch needs that does not depend on the tensors' addresses or the scale."""

    __slots__ = ("generation", "empty", "out_shape", "out_like_q", "head_dim", "pad_dim", "width",
                 "copy", "args", "kernel", "chunk", "ws_bytes", "sync_mode", "device",
                 "device_index", "dtype")


_PLANS: dict[tuple, _LaunchPlan] = {}
_PLANS_MAX = 512


def _device_index(torch_mod, t) -> int:
    return t.device.index if t.device.index is not None else torch_mod.cuda.current_device()


def _raw_stream(torch_mod, device_index: int) -> int:
    get_raw = getattr(torch_mod._C, "_cuda_getCurrentRawStream", None)
    if get_raw is not None:
        return int(get_raw(device_index))
    return int(torch_mod.cuda.current_stream(device_index).cuda_stream)


def _call_knobs(tile: tuple[int, int] | None = None, accum: str | None = None) -> _lib.CallKnobs:
    """The knob values of a call as ``ta_call_knobs`` (the library's ``ta_plan_call``):
    parsed from the ``TILEDATTN_*`` environment exactly as this module parses them, with
    ``tile`` / ``accum`` taking the place of the tile and accumulation knobs when given."""
    k = _lib.CallKnobs()
    if tile is not None:
        k.tile_m, k.tile_n = int(tile[0]), int(tile[1])
    elif os.getenv("TILEDATTN_TILE_M") or os.getenv("TILEDATTN_TILE_N"):
        k.tile_m, k.tile_n = _resolve_tile_config()
    if accum is None:
        raw = (os.getenv("TILEDATTN_ACCUM_MODE") or "").strip().lower()
        accum = None if raw in ("", "auto") else _resolve_accum_mode(seq_len=0, head_dim=0, causal=False)
    k.accum = -1 if accum is None else (_lib.TA_ACC_INPUT if accum == "fp16" else _lib.TA_ACC_FP32)
    k.aligned = 0 if _aligned_fastpath_disabled() else 1
    raw = os.getenv("TILEDATTN_SCHED", "").strip()
    k.sched = -1 if raw == "" else int(raw)
    raw = os.getenv("TILEDATTN_SPLIT", "").strip().lower()
    k.split = (_lib.TA_SPLIT_AUTO if raw in ("", "auto") else 0 if raw in ("0", "off")
               else _lib.TA_SPLIT_PAIRS if raw == "pairs" else int(raw))
    return k


class _CallPolicy:
    """The resolved policy of one call, independent of tensor addresses and strides."""

    __slots__ = ("accum_mode", "accum_code", "tile_m", "tile_n", "explicit_tile", "chunk_plan",
                 "kernel_head_dim", "pad_dim", "pad_in_kernel", "width", "aligned", "sched", "chunk",
                 "ws_bytes")


def _resolve_call(lib, *, batch: int, heads: int, seq_len: int, head_dim: int, dtype_code: int,
                  causal: bool, compute_units: int, tile: tuple[int, int] | None = None,
                  accum: str | None = None, device_index: int = 0) -> _CallPolicy:
    """Knobs and policies of a call (flash_fwd.py:821-921) for a device of ``compute_units``
    CUs: accumulation, tile, kernel head dim and padding, aligned fast path, workgroup order
    and split.  Needs no tensors and no device.  The library's ``ta_plan_call`` applies the
    same rules for callers outside Python (the C++ operator); tests compare the two."""
    if accum is not None:
        if accum not in ("fp32", "fp16"):
            raise ValueError(f"Unsupported accumulation mode {accum!r}. Use fp32 or fp16.")
        accum_mode = accum
    else:
        accum_mode = _resolve_accum_mode(seq_len=seq_len, head_dim=head_dim, causal=causal)
    bh = batch * heads
    pol = _CallPolicy()
    pol.accum_mode = accum_mode
    pol.explicit_tile = tile is not None or bool(os.getenv("TILEDATTN_TILE_M") or os.getenv("TILEDATTN_TILE_N"))
    if tile is not None:
        tile_m, tile_n = int(tile[0]), int(tile[1])
        _check_tile_supported(tile_m, tile_n)
    elif pol.explicit_tile:
        tile_m, tile_n = _resolve_tile_config()
        _check_tile_supported(tile_m, tile_n)
    else:
        tile_m, tile_n = _default_tile_config_for_shape_gfx950(
            seq_len=seq_len, head_dim=head_dim, causal=causal, n_bh=bh, accum_mode=accum_mode,
            compute_units=compute_units,
        )
        # Keep 128 rows where the 128-row kernel would split key ranges, unless the 64-row
        # grid fills at most half the CUs: there the 64-row kernel, whole or split by its own
        # plan, is faster (B1 H1 S2048 causal D = 128: 128-row split 20.0 us, 64-row whole
        # 17.0, 64-row chunks of 4 steps 13.2; B1 H2 S8192, 256 blocks of 64 rows: the
        # 128-row plan 47.2 against 53.9 for the best 64-row split).
        small64 = 2 * bh * ((seq_len + 63) // 64) <= compute_units
        raw_split = os.getenv("TILEDATTN_SPLIT", "").strip().lower()
        if (tile_m == 64 and not (small64 and raw_split in ("", "auto"))
                and _split_preferred(lib, batch, heads, seq_len, head_dim, causal, compute_units, accum_mode)):
            tile_m = 128

    pol.chunk_plan = _resolve_chunk_plan(head_dim)
    kernel_head_dim, pad_dim = _resolve_kernel_head_dim_gfx950(
        head_dim, native_96=tile_n in (64, 128) and accum_mode == "fp32")
    if kernel_head_dim > 128 and tile_n != _WIDE_HEAD_DIM_TILE_N:
        if pol.explicit_tile:
            raise ValueError(
                f"TILEDATTN_TILE_N={tile_n} is not supported for head dimension D={head_dim} "
                f"on gfx950: head dims above 128 run with TILE_N=64."
            )
        tile_n = _WIDE_HEAD_DIM_TILE_N
    accum_code = _lib.TA_ACC_INPUT if accum_mode == "fp16" else _lib.TA_ACC_FP32
    # A narrower head dim that is a multiple of 8 runs in place on the eight-wave kernel
    # (ta_fwd_args.d_real: missing columns read as zero, not written); others are zero-padded
    # on the host as the reference does (flash_fwd.py:868-872) and the output is sliced.
    pol.pad_in_kernel = pad_dim > 0 and head_dim % 8 == 0 and _eight_wave_kernel(
        tile_m=tile_m, tile_n=tile_n, accum_code=accum_code, kernel_head_dim=kernel_head_dim)
    pol.pad_dim = pad_dim
    pol.width = head_dim if pol.pad_in_kernel else kernel_head_dim
    pol.tile_m, pol.tile_n, pol.kernel_head_dim, pol.accum_code = tile_m, tile_n, kernel_head_dim, accum_code
    pol.aligned = int(_use_unmasked_tail_kernel(seq_len=seq_len, tile_m=tile_m, tile_n=tile_n))
    n_qblk = (seq_len + tile_m - 1) // tile_m
    pol.sched = _resolve_sched(n_blocks=bh * n_qblk, causal=causal, tile_m=tile_m, tile_n=tile_n,
                               accum_code=accum_code, head_dim=kernel_head_dim, compute_units=compute_units)
    pol.chunk, pol.ws_bytes = 0, 0
    if bh == 0 or seq_len == 0:
        return pol
    args = _lib.shape_args(B=batch, H=heads, S=seq_len, D=kernel_head_dim, causal=causal, dtype=dtype_code,
                           tile_m=tile_m, tile_n=tile_n, accum=accum_code, sched=pol.sched,
                           aligned=pol.aligned, d_real=head_dim if pol.pad_in_kernel else 0,
                           device=device_index)
    capable = _split_capable(tile_m=tile_m, tile_n=tile_n, accum_code=accum_code,
                             kernel_head_dim=kernel_head_dim)
    pol.chunk = _resolve_split(lib, args, capable=capable, compute_units=compute_units)
    if pol.chunk:
        ws_bytes = ctypes.c_int64(0)
        _raise_for_status(lib, lib.ta_split_workspace_size(ctypes.byref(args), pol.chunk,
                                                           ctypes.byref(ws_bytes)))
        pol.ws_bytes = int(ws_bytes.value)
        if pol.ws_bytes and not os.getenv("TILEDATTN_SCHED", "").strip():
            pol.sched = 1  # the split grid regroups per XCD whenever it divides evenly
    return pol


def _build_plan(torch_mod, lib, q, k, v, causal: bool, tile: tuple[int, int] | None = None,
                accum: str | None = None) -> _LaunchPlan:
    """Resolve knobs and policies for a call (flash_fwd.py:821-969), up to the launch.
    ``tile`` / ``accum`` ('fp32' | 'fp16'), when given, take the place of the
    ``TILEDATTN_TILE_M/N`` and ``TILEDATTN_ACCUM_MODE`` knobs (the operator's arguments)."""
    opt_level, occupancy, num_ctas = _resolve_kernel_options()
    sync_mode = _resolve_sync_mode()

    batch, heads, seq_len, head_dim = map(int, q.shape)
    dtype_code = _dtype_code_for_torch_dtype(q.dtype)
    device_index = _device_index(torch_mod, q)
    pol = _resolve_call(lib, batch=batch, heads=heads, seq_len=seq_len, head_dim=head_dim,
                        dtype_code=dtype_code, causal=causal, tile=tile, accum=accum,
                        compute_units=_compute_units(torch_mod, device_index), device_index=device_index)
    tile_m, tile_n, kernel_head_dim, width = pol.tile_m, pol.tile_n, pol.kernel_head_dim, pol.width

    plan = _LaunchPlan()
    plan.generation = _compile_cache.generation()
    plan.device = q.device
    plan.dtype = q.dtype
    plan.head_dim = head_dim
    plan.pad_dim = 0 if pol.pad_in_kernel else pol.pad_dim
    plan.width = width
    plan.out_shape = (batch, heads, seq_len, width)
    plan.out_like_q = width == head_dim
    plan.sync_mode = sync_mode
    plan.empty = batch * heads == 0 or seq_len == 0
    if plan.empty:
        return plan

    aligned = pol.aligned
    if pol.chunk_plan is not None:
        kernel_variant = "chunked"
    elif aligned:
        kernel_variant = "direct_aligned"
    else:
        kernel_variant = "direct"
    plan.device_index = device_index

    kernel_key = (
        tile_m,
        tile_n,
        kernel_head_dim,
        kernel_variant,
        str(q.dtype),
        causal,
        pol.accum_mode,
        opt_level,
        occupancy if occupancy is not None else -1,
        num_ctas if num_ctas is not None else -1,
        aligned,
        device_index,
    )
    config = (dtype_code, kernel_head_dim, tile_m, tile_n, int(causal), pol.accum_code, aligned)
    plan.kernel = get_kernel(kernel_key, lambda: _Launcher(lib, device_index, config))

    # Which inputs the kernel cannot read in place (host padding or strides); addresses are
    # checked per call.
    plan.copy = tuple(plan.pad_dim > 0 or not _strides_ok(t.stride(), t.shape, width)
                      for t in (q, k, v))
    args = _lib.shape_args(B=batch, H=heads, S=seq_len, D=kernel_head_dim, causal=causal, dtype=dtype_code,
                           tile_m=tile_m, tile_n=tile_n, accum=pol.accum_code, sched=pol.sched,
                           aligned=aligned, d_real=head_dim if pol.pad_in_kernel else 0,
                           device=device_index)
    contiguous = (heads * seq_len * width, seq_len * width, width, 1)
    for name, t, cp in (("q_stride", q, plan.copy[0]), ("k_stride", k, plan.copy[1]),
                        ("v_stride", v, plan.copy[2])):
        getattr(args, name)[:] = contiguous if cp else tuple(t.stride())
    args.o_stride[:] = contiguous
    plan.chunk = pol.chunk
    plan.ws_bytes = pol.ws_bytes
    plan.args = args
    return plan


def _plan_for(torch_mod, q, k, v, causal: bool, tile, accum) -> _LaunchPlan:
    """The cached launch plan of a call (built on the first call of a configuration)."""
    key = (q.shape, q.stride(), k.stride(), v.stride(), q.dtype, q.device, causal, _knob_snapshot(),
           tile, accum)
    plan = _PLANS.get(key)
    if plan is None or plan.generation != _compile_cache.generation():
        plan = _build_plan(torch_mod, _runtime.get_native_library(), q, k, v, causal, tile, accum)
        if len(_PLANS) >= _PLANS_MAX:
            _PLANS.clear()
        _PLANS[key] = plan
    return plan


def describe_call(q, k, v, *, causal: bool, tile: tuple[int, int] | None = None,
                  accum: str | None = None) -> dict:
    """What ``run_flash_fwd`` enqueues for these inputs under the current knobs, as the
    library reports it (``ta_describe_launch``: kernel and code object, grid, layout, split,
    merge kernel, workspace); an empty dict when nothing is launched (zero-size inputs).
    Launches nothing."""
    torch_mod = _runtime.get_torch_module()
    plan = _plan_for(torch_mod, q, k, v, causal, tile, accum)
    if plan.empty:
        return {}
    lib = _runtime.get_native_library()
    return _lib.describe(lib, plan.args, plan.chunk).as_dict()


def run_flash_fwd(
    q,
    k,
    v,
    *,
    causal: bool,
    scale: float,
    tile: tuple[int, int] | None = None,
    accum: str | None = None,
):
    """Run the gfx950 SDPA forward on validated [B,H,S,D] fp16/bf16 tensors; returns o.

    Follows flash_fwd.py:821-973: resolve knobs, pad the head dim if needed (in the kernel
    where it can, else on the host), allocate the output, pick the kernel through the cache,
    launch, apply the sync mode, and return ``[B,H,S,D]`` (a view sliced back to D when
    padded on the host).  K is read row-major in place; no
    transposed view or per-call copy is made unless the inputs' strides require one.  The
    resolution is cached per configuration and knob values (``_build_plan``); a call then
    allocates the output, fills the tensor addresses and scale, and launches.

    ``tile`` (TILE_M, TILE_N) and ``accum`` ('fp32' | 'fp16'), when given, override the
    corresponding knobs (the custom operator passes its arguments this way); ``sdpa`` leaves
    them unset, as the reference's call does.
    """
    torch_mod = _runtime.get_torch_module()
    plan = _plan_for(torch_mod, q, k, v, causal, tile, accum)

    if plan.out_like_q and type(q) is torch_mod.Tensor:
        out = torch_mod.empty_like(q, memory_format=torch_mod.contiguous_format)
    else:
        out = torch_mod.empty(plan.out_shape, dtype=plan.dtype, device=plan.device)
    if not plan.empty:
        wd, pad = plan.width, plan.pad_dim
        qp, kp, vp = q.data_ptr(), k.data_ptr(), v.data_ptr()
        args = _lib.FwdArgs.from_buffer_copy(plan.args)
        if plan.copy[0] or plan.copy[1] or plan.copy[2] or (qp | kp | vp) % 16:
            qk = _kernel_ready(torch_mod, q, wd, pad) if plan.copy[0] or qp % 16 else q
            kk = _kernel_ready(torch_mod, k, wd, pad) if plan.copy[1] or kp % 16 else k
            vk = _kernel_ready(torch_mod, v, wd, pad) if plan.copy[2] or vp % 16 else v
            for name, t in (("q_stride", qk), ("k_stride", kk), ("v_stride", vk)):
                getattr(args, name)[:] = tuple(t.stride())
            qp, kp, vp = qk.data_ptr(), kk.data_ptr(), vk.data_ptr()
        args.q, args.k, args.v, args.o = qp, kp, vp, out.data_ptr()
        args.scale = scale
        if plan.sync_mode == "strict":
            torch_mod.cuda.synchronize(plan.device)
        stream = _raw_stream(torch_mod, plan.device_index)
        if plan.ws_bytes:
            # torch's caching allocator returns 512-byte aligned blocks, stream-ordered: the
            # block is reused only by work enqueued after this launch on the same stream.
            workspace = torch_mod.empty(plan.ws_bytes, dtype=torch_mod.uint8, device=plan.device)
            plan.kernel.split(args, plan.chunk, workspace.data_ptr(), plan.ws_bytes, stream)
        else:
            plan.kernel(args, stream)
        if plan.sync_mode in {"strict", "post"}:
            torch_mod.cuda.current_stream(plan.device).synchronize()

    return out[..., :plan.head_dim] if plan.pad_dim > 0 else out

