"""ctypes binding of libhcg_gfx950.so (the C ABI in include/hcg_gemm.h).

The library is built in-tree by 5_amd/csrc/build.py.  There is no fallback:
if it is missing or cannot be loaded, every gfx950 launch raises
``BackendError``.

torch (when importable) is imported before the library is opened so that
both share one HIP runtime: torch ships its own libamdhip64.so.7 and the
dynamic loader reuses an already-loaded SONAME.
"""

from __future__ import annotations

import ctypes
import os
import threading

from .._errors import BackendError, LaunchError

LIB_NAME = "libhcg_gfx950.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

HCG_OK = 0
HCG_EINVAL = 1
HCG_EHIP = 2

HCG_F16 = 0
HCG_BF16 = 1

HCG_ALGO_AUTO = 0
HCG_ALGO_TILED = 1
HCG_ALGO_SKINNY = 2
HCG_ALGO_GENERIC = 3
HCG_ALGO_TILED_256x256 = 4
HCG_ALGO_TILED_256x192 = 5
HCG_ALGO_TILED_128x256 = 6
HCG_ALGO_TILED_128x128 = 7
HCG_ALGO_TILED_256x64 = 8
HCG_ALGO_NARROW = 9

ALGOS = {
    "auto": HCG_ALGO_AUTO,
    "tiled": HCG_ALGO_TILED,
    "skinny": HCG_ALGO_SKINNY,
    "generic": HCG_ALGO_GENERIC,
    "tiled_256x256": HCG_ALGO_TILED_256x256,
    "tiled_256x192": HCG_ALGO_TILED_256x192,
    "tiled_128x256": HCG_ALGO_TILED_128x256,
    "tiled_128x128": HCG_ALGO_TILED_128x128,
    "tiled_256x64": HCG_ALGO_TILED_256x64,
    "narrow": HCG_ALGO_NARROW,
}

# Every symbol include/hcg_gemm.h, include/hcg_tile_ops.h and include/hcg_mfma.h declare.
EXPORTS = ("hcg_init", "hcg_gemm", "hcg_gemm_algo", "hcg_gemm_noalloc", "hcg_last_error", "hcg_version",
           "hcg_operand_in_place", "hcg_tile_load", "hcg_tile_store", "hcg_mfma_step")

NOALLOC_SCRATCH_BYTES = 32 << 20  # HCG_NOALLOC_SCRATCH_BYTES

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def _declare(lib: ctypes.CDLL) -> None:
    i64 = ctypes.c_int64
    vp = ctypes.c_void_p
    c_int = ctypes.c_int
    lib.hcg_init.argtypes = []
    lib.hcg_init.restype = c_int
    lib.hcg_gemm.argtypes = [c_int, vp, i64, vp, i64, vp, i64, i64, i64, i64, vp]
    lib.hcg_gemm.restype = c_int
    lib.hcg_gemm_algo.argtypes = [c_int, c_int, vp, i64, vp, i64, vp, i64, i64, i64, i64, vp]
    lib.hcg_gemm_algo.restype = c_int
    lib.hcg_gemm_noalloc.argtypes = [c_int, vp, i64, vp, i64, vp, i64, i64, i64, i64, vp]
    lib.hcg_gemm_noalloc.restype = c_int
    lib.hcg_last_error.argtypes = []
    lib.hcg_last_error.restype = ctypes.c_char_p
    lib.hcg_version.argtypes = []
    lib.hcg_version.restype = c_int
    lib.hcg_operand_in_place.argtypes = [vp, i64, i64, i64]
    lib.hcg_operand_in_place.restype = c_int
    u64 = ctypes.c_uint64
    lib.hcg_tile_load.argtypes = [c_int, vp, i64, i64, i64, vp, i64, i64, i64, vp, u64, vp, vp, vp]
    lib.hcg_tile_load.restype = c_int
    lib.hcg_tile_store.argtypes = [c_int, vp, i64, i64, i64, vp, i64, i64, i64, vp, vp, vp]
    lib.hcg_tile_store.restype = c_int
    lib.hcg_mfma_step.argtypes = [c_int, c_int, c_int, c_int, vp, vp, vp, vp, vp, vp, vp]
    lib.hcg_mfma_step.restype = c_int


def load() -> ctypes.CDLL:
    """Open the library once (no device work happens here)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise BackendError(
                f"gfx950 backend library {LIB_PATH} is not built; run 5_amd/csrc/build.py"
            )
        try:
            import torch  # noqa: F401  (share torch's HIP runtime)
        except ImportError:
            pass
        try:
            lib = ctypes.CDLL(LIB_PATH)
        except OSError as exc:
            raise BackendError(f"cannot load {LIB_PATH}: {exc}") from exc
        _declare(lib)
        # Loading leaves the process's garbage collector as it was.  (Its
        # first full collection after torch is imported scans ~170k objects
        # and stops the host for 40-50 ms a few hundred calls in; a caller
        # that minds runs gc.collect() and gc.freeze() once after its imports,
        # as bench.py does.)
        _lib = lib
        return lib


def last_error(lib: ctypes.CDLL) -> str:
    raw = lib.hcg_last_error()
    return raw.decode("utf-8", "replace") if raw else ""


def check(lib: ctypes.CDLL, rc: int, what: str) -> None:
    if rc == HCG_OK:
        return
    msg = last_error(lib)
    if rc == HCG_EINVAL:
        raise LaunchError(f"{what}: {msg}")
    raise BackendError(f"{what} failed ({rc}): {msg}")


def lib() -> ctypes.CDLL:
    """The loaded library (loading it on first use)."""
    return _lib if _lib is not None else load()


def gemm(
    algo: int,
    dtype: int,
    a_ptr: int,
    lda: int,
    b_ptr: int,
    ldb: int,
    c_ptr: int,
    ldc: int,
    m: int,
    n: int,
    k: int,
    stream: int,
) -> None:
    lib = _lib if _lib is not None else load()
    rc = lib.hcg_gemm_algo(algo, dtype, a_ptr, lda, b_ptr, ldb, c_ptr, ldc, m, n, k, stream or None)
    check(lib, rc, "hcg_gemm")


def tile_load(elem_bytes: int, src: int, ld: int, rows: int, cols: int, origins: int, ntiles: int, th: int,
              tw: int, in_mask: int, fill_bits: int, out: int, out_mask: int, stream: int) -> None:
    lib = load()
    rc = lib.hcg_tile_load(elem_bytes, src or None, ld, rows, cols, origins or None, ntiles, th, tw,
                           in_mask or None, fill_bits, out or None, out_mask or None, stream or None)
    check(lib, rc, "hcg_tile_load")


def tile_store(elem_bytes: int, dst: int, ld: int, rows: int, cols: int, origins: int, ntiles: int, th: int,
               tw: int, tiles: int, tile_mask: int, stream: int) -> None:
    lib = load()
    rc = lib.hcg_tile_store(elem_bytes, dst or None, ld, rows, cols, origins or None, ntiles, th, tw,
                            tiles or None, tile_mask or None, stream or None)
    check(lib, rc, "hcg_tile_store")


def mfma_step(dtype: int, m: int, n: int, k: int, a: int, b: int, a_mask: int, b_mask: int, acc_in: int,
              acc_out: int, stream: int) -> None:
    lib = load()
    rc = lib.hcg_mfma_step(dtype, m, n, k, a or None, b or None, a_mask or None, b_mask or None, acc_in or None,
                           acc_out or None, stream or None)
    check(lib, rc, "hcg_mfma_step")
