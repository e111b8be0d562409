"""ctypes binding of the C ABI in ``include/tiledattn.h`` (``libtiledattn.so``).

The library and the gfx950 code objects it loads are built in-tree by
``tiledattention_amd/csrc/build.py`` into ``tiledattention_amd/lib/`` (the native package
beside this one; located without importing it).  ``TILEDATTN_LIB_DIR`` overrides where both
are looked up.  Nothing here falls back to another implementation: if the library is
missing, ``load()`` raises ``DependencyError``.
"""

from __future__ import annotations

import ctypes
import importlib.util
import os
from pathlib import Path
from threading import Lock

from ._errors import DependencyError

ABI_VERSION = 3

TA_OK = 0
TA_EINVAL = 1
TA_EUNSUPPORTED = 2
TA_ENOKERNEL = 3
TA_EHIP = 4

TA_FP16 = 0
TA_BF16 = 1
TA_ACC_FP32 = 0
TA_ACC_INPUT = 1
TA_SPLIT_PAIRS = -1  # chunk length of the paired split

TILE_SHAPES = ((64, 64), (64, 128), (128, 64), (128, 128))
STATIC_SCRATCH_BYTES = 64 << 20  # TA_STATIC_SCRATCH_BYTES


def uses_pairs(*, causal: bool, head_dim: int, tile_m: int, tile_n: int, accum: int, n_bh: int,
               n_qblk: int, sched: int, compute_units: int) -> bool:
    """Whether a whole-row launch runs causal query blocks in pairs; the same rule as
    use_pairs() in csrc/tiledattn.cpp."""
    if not causal or n_qblk < 2 or head_dim > 128:
        return False
    if not (tile_m == 128 and tile_n in (64, 128) and accum == TA_ACC_FP32):
        return False
    if sched == 3:
        return True
    return sched == 1 and n_bh * n_qblk >= 2 * compute_units


def eight_wave_family(*, tile_m: int, tile_n: int, accum: int, head_dim: int) -> bool:
    """The eight-wave kernels (attn_fwd_pp.hsaco): fp32 accumulation with tiles (128, 64) /
    (128, 128) or (64, 64) / (64, 128) at D = 64, 96, 128 or 160; input-dtype
    accumulation with any tile at D = 64 or 128.  The same rule as eight_wave_family() in
    csrc/tiledattn.cpp."""
    if tile_n not in (64, 128) or tile_m not in (64, 128):
        return False
    if accum != TA_ACC_FP32:  # input-dtype accumulation: ta_fwd_ppl_* / ta_fwd_ppl64_*
        return head_dim in (64, 128)
    return (tile_m == 128 and head_dim <= 160) or (tile_m == 64 and head_dim in (64, 96, 128, 160))


def tail_masked(*, seq_len: int, tile_m: int, tile_n: int, accum: int, head_dim: int,
                aligned: bool = True) -> bool:
    """Whether the C ABI launches the tail-masked variant; unmasked_tail() in
    csrc/tiledattn.cpp: S a multiple of both tiles (and of the 128-key step on the
    eight-wave kernels) and the aligned fast path allowed."""
    steps = not eight_wave_family(tile_m=tile_m, tile_n=tile_n, accum=accum, head_dim=head_dim) \
        or seq_len % 128 == 0
    return not (aligned and seq_len % tile_m == 0 and seq_len % tile_n == 0 and steps)


def uses_rows256(*, causal: bool, head_dim: int, tile_m: int, tile_n: int, accum: int, n_bh: int,
                 seq_len: int, compute_units: int) -> bool:
    """Whether a whole-row launch runs 256-row blocks (ta_fwd_pp256_*); the same rule as
    use_rows256() in csrc/tiledattn.cpp."""
    return (not causal and tile_m == 128 and tile_n in (64, 128) and accum == TA_ACC_FP32
            and head_dim in (64, 128) and n_bh * -(-seq_len // 256) >= 2 * compute_units)


def kernel_symbol(*, dtype: int, head_dim: int, tile_m: int, tile_n: int, causal: bool,
                  tail: bool, accum: int, split: bool = False, pair: bool = False,
                  rows256: bool = False) -> tuple[str, str]:
    """(code object file, kernel symbol) the C ABI launches for a configuration; the same
    rule as kernel_id() in csrc/tiledattn.cpp (used to label measurements).  ``split``
    names the split-key-range kernel (its merge kernel is ta_fwd_merge_<dt>_d<D>_c<c>),
    ``pair`` the causal pair kernel (``uses_pairs``); both together the paired-split
    kernel; ``rows256`` the 256-row kernel (``uses_rows256``; its tail variant also runs
    when S is not a multiple of 256).  ``tail`` is the variant the C ABI picks
    (``tail_masked``)."""
    dt = "bf16" if dtype == TA_BF16 else "f16"
    c, t = int(bool(causal)), int(bool(tail))
    if rows256:
        if causal or head_dim not in (64, 128) or accum != TA_ACC_FP32 or tile_m != 128:
            raise ValueError("256-row blocks exist for non-causal fp32 D = 64 / 128 at 128-row tiles")
        return "attn_fwd_pp.hsaco", f"ta_fwd_pp256_{dt}_d{head_dim}_c0_t{t}"
    if tile_m == 128 and tile_n in (64, 128) and accum == TA_ACC_FP32 and head_dim <= 160:
        kind = ("pp_psplit" if pair else "pp_split") if split else ("pp_pair" if pair else "pp")
        return "attn_fwd_pp.hsaco", f"ta_fwd_{kind}_{dt}_d{head_dim}_c{c}_t{t}"
    if (eight_wave_family(tile_m=tile_m, tile_n=tile_n, accum=accum, head_dim=head_dim)
            and not split and not pair):
        if accum == TA_ACC_FP32:
            return "attn_fwd_pp.hsaco", f"ta_fwd_pp64_{dt}_d{head_dim}_c{c}_t{t}"
        kind = f"{'ppl' if tile_m == 128 else 'ppl64'}_n{tile_n}"
        return "attn_fwd_pp.hsaco", f"ta_fwd_{kind}_{dt}_d{head_dim}_c{c}_t{t}"
    if split:
        raise ValueError("split key ranges exist for tiles (128, 64) and (128, 128), fp32 "
                         "accumulation, D <= 160")
    return (f"attn_fwd_m{tile_m}_n{tile_n}.hsaco",
            f"ta_fwd_{dt}_d{head_dim}_m{tile_m}_n{tile_n}_c{c}_t{t}_a{int(accum != TA_ACC_FP32)}")

# Every symbol the header declares; tests check the built library exports all of them.
EXPORTED_SYMBOLS = (
    "ta_abi_version",
    "ta_set_code_object_dir",
    "ta_prepare",
    "ta_sdpa_fwd",
    "ta_split_plan",
    "ta_split_plan_model",
    "ta_split_workspace_size",
    "ta_sdpa_fwd_split",
    "ta_sdpa_fwd_split_static",
    "ta_cache_reset",
    "ta_cache_size",
    "ta_last_error",
    "ta_status_string",
)


class FwdArgs(ctypes.Structure):
    """Mirror of ``ta_fwd_args``."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("B", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("S", ctypes.c_int64),
        ("D", ctypes.c_int64),
        ("q_stride", ctypes.c_int64 * 4),
        ("k_stride", ctypes.c_int64 * 4),
        ("v_stride", ctypes.c_int64 * 4),
        ("o_stride", ctypes.c_int64 * 4),
        ("scale", ctypes.c_float),
        ("causal", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("tile_m", ctypes.c_int32),
        ("tile_n", ctypes.c_int32),
        ("accum", ctypes.c_int32),
        ("device", ctypes.c_int32),
        ("sched", ctypes.c_int32),
        ("d_real", ctypes.c_int32),
        ("aligned", ctypes.c_int32),
    ]


_lock = Lock()
_lib: ctypes.CDLL | None = None


def lib_dir() -> Path:
    """Directory of ``libtiledattn.so`` and the code objects: ``TILEDATTN_LIB_DIR``, else
    ``lib/`` beside this package (a kernel package laid out by
    ``tiledattention_amd.kernel_build`` carries its own), else ``lib/`` of the
    ``tiledattention_amd`` package (found by its import spec, which does not execute it)."""
    env = os.getenv("TILEDATTN_LIB_DIR", "").strip()
    if env:
        return Path(env)
    own = Path(__file__).resolve().parent / "lib"
    if (own / "libtiledattn.so").exists():
        return own
    spec = importlib.util.find_spec("tiledattention_amd")
    if spec is None or not spec.submodule_search_locations:
        raise DependencyError(
            "The native package tiledattention_amd (kernels and C-ABI library) is not installed."
        )
    return Path(list(spec.submodule_search_locations)[0]) / "lib"


def library_path() -> Path:
    return lib_dir() / "libtiledattn.so"


def code_object_paths() -> list[Path]:
    d = lib_dir()
    return [d / f"attn_fwd_m{tm}_n{tn}.hsaco" for tm, tn in TILE_SHAPES] + [d / "attn_fwd_pp.hsaco"]


def _declare(lib: ctypes.CDLL) -> None:
    i32 = ctypes.c_int32
    lib.ta_abi_version.argtypes = []
    lib.ta_abi_version.restype = ctypes.c_int
    lib.ta_set_code_object_dir.argtypes = [ctypes.c_char_p]
    lib.ta_set_code_object_dir.restype = i32
    lib.ta_prepare.argtypes = [i32, i32, i32, i32, i32, i32, i32, i32]
    lib.ta_prepare.restype = i32
    lib.ta_sdpa_fwd.argtypes = [ctypes.POINTER(FwdArgs), ctypes.c_void_p]
    lib.ta_sdpa_fwd.restype = i32
    lib.ta_split_plan.argtypes = [ctypes.POINTER(FwdArgs), ctypes.POINTER(i32)]
    lib.ta_split_plan.restype = i32
    lib.ta_split_plan_model.argtypes = [ctypes.c_int64, ctypes.c_int64, i32, i32]
    lib.ta_split_plan_model.restype = i32
    lib.ta_split_workspace_size.argtypes = [ctypes.POINTER(FwdArgs), i32, ctypes.POINTER(ctypes.c_int64)]
    lib.ta_split_workspace_size.restype = i32
    lib.ta_sdpa_fwd_split.argtypes = [ctypes.POINTER(FwdArgs), i32, ctypes.c_void_p, ctypes.c_int64,
                                      ctypes.c_void_p]
    lib.ta_sdpa_fwd_split.restype = i32
    lib.ta_sdpa_fwd_split_static.argtypes = [ctypes.POINTER(FwdArgs), i32, ctypes.c_void_p]
    lib.ta_sdpa_fwd_split_static.restype = i32
    lib.ta_cache_reset.argtypes = []
    lib.ta_cache_reset.restype = i32
    lib.ta_cache_size.argtypes = []
    lib.ta_cache_size.restype = i32
    lib.ta_last_error.argtypes = []
    lib.ta_last_error.restype = ctypes.c_char_p
    lib.ta_status_string.argtypes = [i32]
    lib.ta_status_string.restype = ctypes.c_char_p


def load() -> ctypes.CDLL:
    """Load the C-ABI library once per process; raise ``DependencyError`` if absent."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            raise DependencyError(
                f"Native library {path} is missing. Build it with "
                "`python -m tiledattention_amd.csrc.build` (needs hipcc for gfx950)."
            )
        missing = [str(p) for p in code_object_paths() if not p.exists()]
        if missing:
            raise DependencyError(
                "gfx950 code objects are missing: " + ", ".join(missing)
                + ". Build them with `python -m tiledattention_amd.csrc.build`."
            )
        try:
            lib = ctypes.CDLL(str(path))
        except OSError as exc:
            raise DependencyError(f"Native library {path} could not be loaded: {exc}") from exc
        _declare(lib)
        ver = int(lib.ta_abi_version())
        if ver != ABI_VERSION:
            raise DependencyError(f"libtiledattn ABI {ver} does not match the binding's {ABI_VERSION}.")
        st = lib.ta_set_code_object_dir(str(lib_dir()).encode())
        if st != TA_OK:
            raise DependencyError(f"ta_set_code_object_dir failed: {last_error(lib)}")
        _lib = lib
        return lib


def loaded() -> ctypes.CDLL | None:
    """The library if ``load()`` already succeeded in this process, else None."""
    return _lib


def last_error(lib: ctypes.CDLL) -> str:
    raw = lib.ta_last_error()
    return raw.decode(errors="replace") if raw else ""


def status_name(lib: ctypes.CDLL, status: int) -> str:
    raw = lib.ta_status_string(int(status))
    return raw.decode() if raw else str(status)


def _reset_for_tests() -> None:
    global _lib
    with _lock:
        _lib = None
