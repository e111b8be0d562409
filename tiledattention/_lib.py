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

ABI_VERSION = 6

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
TA_SPLIT_AUTO = -2   # chunk length chosen by the dispatch model

TILE_SHAPES = ((64, 64), (64, 128), (128, 64), (128, 128))
STATIC_SCRATCH_BYTES = 64 << 20  # TA_STATIC_SCRATCH_BYTES


TA_LAYOUT_WHOLE_ROWS = 0
TA_LAYOUT_PAIRS = 1
TA_LAYOUT_ROWS256 = 2
TA_LAYOUT_SPLIT = 3
TA_LAYOUT_PAIRED_SPLIT = 4
TA_LAYOUT_WIDE = 5


# Every symbol the header declares; tests check the built library exports all of them.
EXPORTED_SYMBOLS = (
    "ta_abi_version",
    "ta_set_code_object_dir",
    "ta_prepare",
    "ta_sdpa_fwd",
    "ta_split_plan",
    "ta_split_plan_model",
    "ta_split_plan_model_rows",
    "ta_split_workspace_size",
    "ta_sdpa_fwd_split",
    "ta_sdpa_fwd_split_static",
    "ta_describe_launch",
    "ta_describe_launch_model",
    "ta_plan_call",
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


class LaunchDesc(ctypes.Structure):
    """Mirror of ``ta_launch_desc``: what one forward enqueues (filled by the library)."""

    _fields_ = [
        ("code_object", ctypes.c_char * 64),
        ("kernel", ctypes.c_char * 96),
        ("grid", ctypes.c_int64),
        ("block", ctypes.c_int32),
        ("rows", ctypes.c_int32),
        ("tail", ctypes.c_int32),
        ("layout", ctypes.c_int32),
        ("chunk_steps", ctypes.c_int32),
        ("compute_units", ctypes.c_int32),
        ("merge_kernel", ctypes.c_char * 96),
        ("merge_grid", ctypes.c_int64),
        ("merge_block", ctypes.c_int32),
        ("in_place_pad", ctypes.c_int32),
        ("split_capable", ctypes.c_int32),
        ("merge_in_kernel", ctypes.c_int32),
        ("workspace_bytes", ctypes.c_int64),
    ]

    def as_dict(self) -> dict:
        out = {}
        for name, _ in self._fields_:
            if name == "reserved":
                continue
            val = getattr(self, name)
            out[name] = val.decode() if isinstance(val, bytes) else int(val)
        return out


class CallKnobs(ctypes.Structure):
    """Mirror of ``ta_call_knobs``."""

    _fields_ = [("tile_m", ctypes.c_int32), ("tile_n", ctypes.c_int32), ("accum", ctypes.c_int32),
                ("aligned", ctypes.c_int32), ("sched", ctypes.c_int32), ("split", ctypes.c_int32)]


class CallPlan(ctypes.Structure):
    """Mirror of ``ta_call_plan``."""

    _fields_ = [("args", FwdArgs), ("chunk_steps", ctypes.c_int32), ("host_pad", ctypes.c_int32),
                ("out_width", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("workspace_bytes", ctypes.c_int64)]


def shape_args(*, B: int = 1, H: int = 1, S: int = 128, D: int = 128, causal: bool = False,
               dtype: int = TA_BF16, tile_m: int = 128, tile_n: int = 64, accum: int = TA_ACC_FP32,
               sched: int = 0, aligned: int = 1, d_real: int = 0, device: int = 0) -> "FwdArgs":
    """A ``FwdArgs`` carrying only the fields the planning queries read (no tensors)."""
    a = FwdArgs()
    a.B, a.H, a.S, a.D = B, H, S, D
    a.causal, a.dtype, a.tile_m, a.tile_n, a.accum = int(causal), dtype, tile_m, tile_n, accum
    a.sched, a.aligned, a.d_real, a.device = sched, aligned, d_real, device
    return a


def describe(lib: ctypes.CDLL, args: "FwdArgs", chunk_steps: int = 0,
             compute_units: int | None = None) -> LaunchDesc:
    """What ``ta_sdpa_fwd`` (chunk 0) or ``ta_sdpa_fwd_split`` would launch for ``args``:
    on ``args.device`` (``ta_describe_launch``), or for a device of ``compute_units`` CUs
    without touching one (``ta_describe_launch_model``).  Raises ``ValueError`` with the
    library's message on a non-OK status."""
    out = LaunchDesc()
    if compute_units is None:
        st = lib.ta_describe_launch(ctypes.byref(args), int(chunk_steps), ctypes.byref(out))
    else:
        st = lib.ta_describe_launch_model(ctypes.byref(args), int(chunk_steps), int(compute_units),
                                          ctypes.byref(out))
    if st != TA_OK:
        raise ValueError(f"{status_name(lib, st)}: {last_error(lib)}")
    return out


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
    return [d / f"attn_fwd_m{tm}_n{tn}.hsaco" for tm, tn in TILE_SHAPES] + [d / "attn_fwd_pp.hsaco",
                                                                            d / "attn_fwd_wide.hsaco"]


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
    lib.ta_split_plan_model_rows.argtypes = [ctypes.c_int64, ctypes.c_int64, i32, i32, i32, i32]
    lib.ta_split_plan_model_rows.restype = i32
    lib.ta_split_workspace_size.argtypes = [ctypes.POINTER(FwdArgs), i32, ctypes.POINTER(ctypes.c_int64)]
    lib.ta_split_workspace_size.restype = i32
    lib.ta_sdpa_fwd_split.argtypes = [ctypes.POINTER(FwdArgs), i32, ctypes.c_void_p, ctypes.c_int64,
                                      ctypes.c_void_p]
    lib.ta_sdpa_fwd_split.restype = i32
    lib.ta_sdpa_fwd_split_static.argtypes = [ctypes.POINTER(FwdArgs), i32, ctypes.c_void_p]
    lib.ta_sdpa_fwd_split_static.restype = i32
    lib.ta_describe_launch.argtypes = [ctypes.POINTER(FwdArgs), i32, ctypes.POINTER(LaunchDesc)]
    lib.ta_describe_launch.restype = i32
    lib.ta_describe_launch_model.argtypes = [ctypes.POINTER(FwdArgs), i32, i32, ctypes.POINTER(LaunchDesc)]
    lib.ta_describe_launch_model.restype = i32
    lib.ta_plan_call.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, i32, i32, i32,
                                 i32, ctypes.POINTER(CallKnobs), ctypes.POINTER(CallPlan)]
    lib.ta_plan_call.restype = i32
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
