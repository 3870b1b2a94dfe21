"""CPU oracle for the hc tiled matrix-core GEMM -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker (or the
timed CPU baseline).  The product path under ``5_amd/`` never imports it.

Semantics restated (reference citations):

* ``wmma_gfx11`` fallback body, examples/amdgpu_gfx11_wmma_matmul.py:177-190:
  per lane ``accum += np.float32(a_tile[r, k]) * np.float32(b_tile[k, col])``
  for k in 0..15, on tiles whose inactive (out-of-bounds) entries were set to
  +0 (``with_inactive``, :178-179, hc/_sim_types.py:353-357).
* The accumulator starts at ``vzeros`` (:249-256) and is threaded through the
  K loop in ascending ``k0`` (:315-324), so the whole launch is one strictly
  sequential float32 fold per output element, k ascending, starting at +0.
* Tile loads give masked-off payload 0 beyond M/N/K (hc/simulator.py:1338-1357)
  and the store writes only the in-bounds part of C (hc/simulator.py:1441-1458).

Parity pins for each function live in tests/test_oracle.py:

* :func:`gemm_sequential` -- against a scalar ``np.float32`` triple loop
  (brute force), against the reference's blocked-sum check within its own
  ``atol=2e-6`` at the reference test shapes, against order-independent
  integer known-answer tests (bit-exact), and against the float64 product
  within the Higham bound ``gamma_K * (|A||B|)``.
* :func:`gemm_c` (the C restatement, oracle/hc_oracle.c) -- bit-exact against
  :func:`gemm_sequential` on random and ragged shapes for fp16 and bf16.
* :func:`f32_to_bf16_bits` -- against torch's round-to-nearest-even cast and
  hand-computed tie cases.
* :func:`parity_check` -- its tolerance arithmetic is checked on planted
  errors (a dropped k term, a transposed operand) that must fail.
* :func:`simulate_lane_structure` -- bit-exact against the scalar triple loop
  (used only to time the reference's CPU path shape).
* :func:`tile_load` / :func:`tile_store` (the masked tile access of
  hc/simulator.py:1304-1357, 1416-1458) -- against per-element brute-force
  loops, against plain numpy slices for interior tiles, and on hand-computed
  edge, fully-outside and masked cases.
"""

from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libhc_oracle.so")

F16 = 0
BF16 = 1


# --------------------------------------------------------------------------
# bf16 helpers (numpy has no bfloat16; values travel as uint16 bit patterns)
# --------------------------------------------------------------------------


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (round-to-nearest-even) as uint16 bits.

    NaN inputs are not expected (the generators draw finite values).  In
    uint32: a finite float32's bits are at most 0xFF7FFFFF, so adding at most
    0x8000 cannot wrap.
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = (u + (0x7FFF + ((u >> 16) & 1))) >> 16
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def operand_to_f32(x: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == F16:
        return np.asarray(x, dtype=np.float16).astype(np.float32)
    return bf16_bits_to_f32(x)


def operand_bits(x: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == F16:
        return np.ascontiguousarray(x, dtype=np.float16).view(np.uint16)
    return np.ascontiguousarray(x, dtype=np.uint16)


# --------------------------------------------------------------------------
# NumPy restatement
# --------------------------------------------------------------------------


def gemm_sequential(a: np.ndarray, b: np.ndarray, dtype: int = F16) -> np.ndarray:
    """C = A @ B as one sequential float32 fold per element, k ascending.

    Follows examples/amdgpu_gfx11_wmma_matmul.py:183-189 (the per-lane MAC),
    :315-324 (ascending K loop) and :249-256 (zero-initialised accumulator).
    Each step rounds the (exact) product and the sum to float32, exactly as
    NumPy scalar float32 arithmetic does in the reference.
    """
    a32 = operand_to_f32(a, dtype)
    b32 = operand_to_f32(b, dtype)
    m, k = a32.shape
    k2, n = b32.shape
    if k != k2:
        raise ValueError("A.shape[1] must match B.shape[0]")
    acc = np.zeros((m, n), dtype=np.float32)
    for kk in range(k):
        prod = a32[:, kk : kk + 1] * b32[kk : kk + 1, :]  # float32, exact
        acc += prod  # float32 round-to-nearest-even, elementwise
    return acc


def gemm_bruteforce(a: np.ndarray, b: np.ndarray, dtype: int = F16) -> np.ndarray:
    """Scalar triple loop with ``np.float32`` scalars; tiny shapes only."""
    a32 = operand_to_f32(a, dtype)
    b32 = operand_to_f32(b, dtype)
    m, k = a32.shape
    _, n = b32.shape
    out = np.zeros((m, n), dtype=np.float32)
    for i in range(m):
        for j in range(n):
            s = np.float32(0.0)
            for kk in range(k):
                s = np.float32(s + np.float32(a32[i, kk]) * np.float32(b32[kk, j]))
            out[i, j] = s
    return out


def gemm_blocked(a: np.ndarray, b: np.ndarray, dtype: int = F16, block: int = 16) -> np.ndarray:
    """Sum over 16-wide K blocks of float32 matrix products.

    This is the check the reference's own test applies to the simulator output
    (tests/test_examples.py:23-33 with the helper at
    examples/amdgpu_gfx11_wmma_matmul.py:329-335, ``atol=2e-6``); its
    summation order differs from the simulator's, so it agrees only to that
    tolerance.
    """
    a32 = operand_to_f32(a, dtype)
    b32 = operand_to_f32(b, dtype)
    out = np.zeros((a32.shape[0], b32.shape[1]), dtype=np.float32)
    for k0 in range(0, a32.shape[1], block):
        out += a32[:, k0 : k0 + block] @ b32[k0 : k0 + block, :]
    return out


def simulate_lane_structure(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """The reference simulator's work structure, for timing its CPU path.

    Walks the launch the way hc.simulator runs tiled_gfx11_wmma_matmul:
    one workgroup per 16x16 C tile in dim-0-fastest order
    (hc/simulator.py:917-931, 1298-1301), a K loop in 16-wide steps
    (examples/amdgpu_gfx11_wmma_matmul.py:315-324) over masked 16x16 tile
    copies (hc/simulator.py:1338-1357), and per step the wave32 lanes'
    fallback MACs: lane l owns column l % 16 and rows l//16, l//16 + 2, ...
    (examples/amdgpu_gfx11_wmma_matmul.py:86-93, 177-190), each an
    np.float32 scalar multiply-add.  Greenlet switching, masks and the
    profile hook are not modelled, so this understates the simulator's
    cost.  fp16 only; small shapes only (one Python MAC per flop pair).
    """
    m, k = a.shape
    _, n = b.shape
    c = np.zeros((m, n), dtype=np.float32)
    a32 = a.astype(np.float32)
    b32 = b.astype(np.float32)
    for gj in range((n + 15) // 16):
        for gi in range((m + 15) // 16):
            r0, c0 = gi * 16, gj * 16
            acc = [[np.float32(0.0)] * 8 for _ in range(32)]
            for k0 in range(0, k, 16):
                at = np.zeros((16, 16), dtype=np.float32)
                bt = np.zeros((16, 16), dtype=np.float32)
                blk_a = a32[r0 : r0 + 16, k0 : k0 + 16]
                blk_b = b32[k0 : k0 + 16, c0 : c0 + 16]
                at[: blk_a.shape[0], : blk_a.shape[1]] = blk_a
                bt[: blk_b.shape[0], : blk_b.shape[1]] = blk_b
                for lane in range(32):
                    col = lane % 16
                    frag = acc[lane]
                    for idx, row in enumerate(range(lane // 16, 16, 2)):
                        s = frag[idx]
                        for kk in range(16):
                            s += at[row, kk] * bt[kk, col]
                        frag[idx] = s
            for lane in range(32):
                col = c0 + lane % 16
                if col >= n:
                    continue
                for idx, row in enumerate(range(lane // 16, 16, 2)):
                    if r0 + row < m:
                        c[r0 + row, col] = acc[lane][idx]
    return c


# --------------------------------------------------------------------------
# C restatement (oracle/hc_oracle.c) through ctypes
# --------------------------------------------------------------------------

_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"oracle library {LIB_PATH} is not built; run oracle/build.py"
            )
        lib = ctypes.CDLL(LIB_PATH)
        i64 = ctypes.c_int64
        vp = ctypes.c_void_p
        lib.hco_gemm.argtypes = [ctypes.c_int, vp, i64, vp, i64, vp, i64, i64, i64, i64, ctypes.c_int]
        lib.hco_gemm.restype = ctypes.c_int
        lib.hco_gemm_rows.argtypes = [
            ctypes.c_int, vp, i64, vp, i64, i64, i64, i64, vp, i64, vp, ctypes.c_int
        ]
        lib.hco_gemm_rows.restype = ctypes.c_int
        lib.hco_to_float.argtypes = [ctypes.c_int, vp, vp, i64]
        lib.hco_to_float.restype = None
        lib.hco_max_threads.argtypes = []
        lib.hco_max_threads.restype = ctypes.c_int
        _LIB = lib
    return _LIB


def available() -> bool:
    return os.path.exists(LIB_PATH)


def default_threads() -> int:
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    return max(1, min(16, os.cpu_count() or 1))


def gemm_c(a: np.ndarray, b: np.ndarray, dtype: int = F16, threads: int | None = None) -> np.ndarray:
    """Full C = A @ B from the C restatement (same bits as gemm_sequential)."""
    ab = operand_bits(a, dtype)
    bb = operand_bits(b, dtype)
    m, k = ab.shape
    k2, n = bb.shape
    if k != k2:
        raise ValueError("A.shape[1] must match B.shape[0]")
    out = np.empty((m, n), dtype=np.float32)
    rc = _lib().hco_gemm(
        dtype, ab.ctypes.data, k, bb.ctypes.data, n, out.ctypes.data, n, m, n, k,
        threads or default_threads(),
    )
    if rc != 0:
        raise RuntimeError(f"hco_gemm failed with {rc}")
    return out


def gemm_c_rows(
    a: np.ndarray, b: np.ndarray, rows: np.ndarray, dtype: int = F16, threads: int | None = None
) -> np.ndarray:
    """Rows ``rows`` of C = A @ B, shape (len(rows), N)."""
    ab = operand_bits(a, dtype)
    bb = operand_bits(b, dtype)
    m, k = ab.shape
    _, n = bb.shape
    r = np.ascontiguousarray(rows, dtype=np.int64)
    out = np.empty((r.size, n), dtype=np.float32)
    rc = _lib().hco_gemm_rows(
        dtype, ab.ctypes.data, k, bb.ctypes.data, n, m, n, k, r.ctypes.data, r.size,
        out.ctypes.data, threads or default_threads(),
    )
    if rc != 0:
        raise RuntimeError(f"hco_gemm_rows failed with {rc}")
    return out


def to_float_c(bits: np.ndarray, dtype: int) -> np.ndarray:
    src = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(src.shape, dtype=np.float32)
    _lib().hco_to_float(dtype, src.ctypes.data, out.ctypes.data, src.size)
    return out


# --------------------------------------------------------------------------
# Parity criterion
# --------------------------------------------------------------------------


@dataclass
class ParityReport:
    rel_fro: float
    max_abs: float
    max_abs_bound: float
    rel_fro_bound: float
    ok: bool

    def __str__(self) -> str:
        return (
            f"rel_fro={self.rel_fro:.3e} (<= {self.rel_fro_bound:.1e}) "
            f"max|err|={self.max_abs:.3e} (<= {self.max_abs_bound:.3e}) ok={self.ok}"
        )


def max_abs_bound(k: int) -> float:
    """max elementwise |err| <= 2e-2 * sqrt(K / 1024)."""
    return 2e-2 * math.sqrt(max(k, 0) / 1024.0)


def parity_check(got: np.ndarray, want: np.ndarray, k: int, rel_fro_bound: float = 1e-3) -> ParityReport:
    """Relative Frobenius error <= 1e-3 and max |err| <= 2e-2*sqrt(K/1024)."""
    g = np.asarray(got, dtype=np.float64)
    w = np.asarray(want, dtype=np.float64)
    if g.shape != w.shape:
        raise ValueError(f"shape mismatch {g.shape} vs {w.shape}")
    if not np.all(np.isfinite(g)):
        return ParityReport(math.inf, math.inf, max_abs_bound(k), rel_fro_bound, False)
    diff = g - w
    denom = float(np.linalg.norm(w))
    num = float(np.linalg.norm(diff))
    rel = num / denom if denom > 0 else (0.0 if num == 0 else math.inf)
    mx = float(np.max(np.abs(diff))) if diff.size else 0.0
    bound = max_abs_bound(k)
    return ParityReport(rel, mx, bound, rel_fro_bound, rel <= rel_fro_bound and mx <= bound)


# --------------------------------------------------------------------------
# Masked tile access (group.load / with_inactive / .mask / group.store)
# --------------------------------------------------------------------------


def tile_load(
    src: np.ndarray, origins: np.ndarray, shape: tuple[int, int], mask: np.ndarray | None = None, fill=0
) -> tuple[np.ndarray, np.ndarray]:
    """Per tile t at origin (r0, c0): ``group.load(src[r0:r0+th, c0:c0+tw],
    shape=(th, tw))`` -- the in-bounds overlap is copied, the rest is
    inactive (``_copy_loaded_value``, hc/simulator.py:1338-1357) -- or with
    ``mask``, active only where the mask is also true (``_load_masked``,
    :1324-1336); then ``with_inactive(fill)`` and ``.mask``
    (doc/langref.md:577-595).  Negative origins count as outside (the
    slice is clipped to the part inside ``src``).  Returns (tiles, active)."""
    th, tw = shape
    origins = np.asarray(origins, dtype=np.int64).reshape(-1, 2)
    n = origins.shape[0]
    out = np.full((n, th, tw), fill, dtype=src.dtype)
    active = np.zeros((n, th, tw), dtype=bool)
    rows, cols = src.shape
    for t, (r0, c0) in enumerate(origins):
        # Tile rows/columns that fall inside src.
        ra, rb = max(0, -r0), min(th, rows - r0)
        ca, cb = max(0, -c0), min(tw, cols - c0)
        if ra >= rb or ca >= cb:
            continue
        out[t, ra:rb, ca:cb] = src[r0 + ra : r0 + rb, c0 + ca : c0 + cb]
        active[t, ra:rb, ca:cb] = True
    if mask is not None:
        active &= np.asarray(mask, dtype=bool)
        out = np.where(active, out, np.array(fill, dtype=src.dtype))
    return out, active


def tile_store(dst: np.ndarray, origins: np.ndarray, tiles: np.ndarray, mask: np.ndarray | None = None) -> None:
    """Per tile t at origin (r0, c0), in tile order: ``group.store(dst[r0:r0+th,
    c0:c0+tw], tile)`` -- within the overlap of the view and the tile, active
    elements are written and nothing else changes (``_store_from_value``,
    hc/simulator.py:1441-1458).  Updates ``dst`` in place."""
    n, th, tw = tiles.shape
    origins = np.asarray(origins, dtype=np.int64).reshape(-1, 2)
    act = np.ones(tiles.shape, dtype=bool) if mask is None else np.asarray(mask, dtype=bool)
    rows, cols = dst.shape
    for t, (r0, c0) in enumerate(origins):
        ra, rb = max(0, -r0), min(th, rows - r0)
        ca, cb = max(0, -c0), min(tw, cols - c0)
        if ra >= rb or ca >= cb:
            continue
        region = dst[r0 + ra : r0 + rb, c0 + ca : c0 + cb]
        sel = act[t, ra:rb, ca:cb]
        region[sel] = tiles[t, ra:rb, ca:cb][sel]
