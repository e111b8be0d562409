"""Native side of the MI355X SDPA forward: the gfx950 HIP kernels and the C-ABI library.

* ``csrc/`` holds the sources (kernels, the ``include/tiledattn.h`` implementation) and the
  build recipe, ``python -m tiledattention_amd.csrc.build``;
* ``lib/`` receives what that recipe builds: ``libtiledattn.so`` and the ``.hsaco`` code
  objects it loads.

The Python API lives in the ``tiledattention`` package, under the reference's module path
(``src/tiledattention/__init__.py:20-55``); it loads this package's library through
``tiledattention._lib``.  Importing ``tiledattention_amd`` re-exports that API unchanged
(the same function and exception objects), for callers written against the earlier name.
"""

from __future__ import annotations

from pathlib import Path

from tiledattention import (  # noqa: F401  (re-exported)
    DependencyError,
    DTypeNotSupportedError,
    InvalidShapeError,
    TiledAttentionError,
    UnsupportedPlatformError,
    __all__,
    __version__,
    sdpa,
)

CSRC_DIR = Path(__file__).resolve().parent / "csrc"
LIB_DIR = Path(__file__).resolve().parent / "lib"
