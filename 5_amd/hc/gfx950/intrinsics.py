"""One wave of a gfx950 matrix-core intrinsic: its fallback body for every
lane, and its ``amdgpu-gfx950`` lowering executed on the GPU.

The reference defines an intrinsic by a fallback body plus per-target
lowerings that "must preserve the observable semantics of the fallback body,
including result type, logical shape, masking, and layout behavior"
(doc/langref.md:894-899; hooks hc/core.py:282-307).  For the intrinsics of
``hc.gfx950.kernels`` (signature ``(group, a_tile, b_tile, acc_frag, *,
lane, wave_size, arch)``) this module makes both sides executable for one
64-lane wave:

* ``fallback_wave`` runs the fallback body once per lane, with the
  simulator's value rules (tiles carry an activity mask; ``with_inactive``
  and reading rules as hc/_sim_types.py:287-357) and the intrinsic's verify
  hook called per lane as hc/simulator.py:972-1001 calls it;
* ``run_wave`` calls the intrinsic's registered ``amdgpu-gfx950`` lowering
  with a recording ``ctx`` (``_lowering``), checks the op it creates against
  the instructions this library executes, and runs that op through
  ``hcg_mfma_step`` (include/hcg_mfma.h): the matrix-core instruction itself,
  on the same tiles and accumulators.

Both return lane-major accumulators, shape (64, m*n/64) float32.  Tiles are
NumPy arrays: float16 values, or bfloat16 as uint16 bits (``dtype=
"bfloat16"``); masks are bool arrays of the tile's shape (None: all active).
"""

from __future__ import annotations

from typing import Any

import numpy as np

from .._errors import LaunchError
from ..core import WorkItem
from . import _native
from ._contract import _CallSig, _Masked
from ._lowering import TARGET_ARCH, LoweringError, check_matrix_op, record_lowering

TARGET = "amdgpu-gfx950"
WAVE = TARGET_ARCH[TARGET][1]


class _WaveGroup:
    """The group handle a fallback body sees: ``vload`` of its result."""

    @staticmethod
    def vload(values: Any, *, shape: Any = None, mask: Any = None, layout: Any = None) -> _Masked:
        data = np.asarray(values)
        if shape is not None:
            data = data.reshape(tuple(int(d) for d in shape))
        active = np.ones(data.shape, dtype=bool) if mask is None else np.asarray(mask, dtype=bool)
        return _Masked(data, active, "vector")


class _Lane:
    """``lane`` as the lowering sees it: a per-lane value, not a constant."""

    def __repr__(self) -> str:
        return "<lane id>"


def _payload(tile: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "float16":
        return np.asarray(tile, dtype=np.float16)
    if dtype == "bfloat16":
        bits = np.asarray(tile, dtype=np.uint16)
        return (bits.astype(np.uint32) << 16).view(np.float32)
    raise LaunchError(f"dtype must be 'float16' or 'bfloat16', got {dtype!r}")


def _mask(mask: np.ndarray | None, shape: tuple[int, ...], what: str) -> np.ndarray:
    if mask is None:
        return np.ones(shape, dtype=bool)
    mask = np.asarray(mask)
    if mask.shape != shape or mask.dtype != np.dtype(bool):
        raise LaunchError(f"{what} mask must be a bool array of shape {shape}, got {mask.dtype} {mask.shape}")
    return mask


def _lane_args(a: np.ndarray, b: np.ndarray, acc: np.ndarray, dtype: str, a_mask: Any, b_mask: Any
               ) -> tuple[_Masked, _Masked, list[_Masked]]:
    a_tile = _Masked(_payload(a, dtype), _mask(a_mask, np.shape(a), "A"), "tensor")
    b_tile = _Masked(_payload(b, dtype), _mask(b_mask, np.shape(b), "B"), "tensor")
    acc = np.asarray(acc, dtype=np.float32)
    if acc.ndim != 2 or acc.shape[0] != WAVE:
        raise LaunchError(f"accumulators must be ({WAVE}, registers) float32, got {acc.shape}")
    frags = [_Masked(acc[lane].copy(), np.ones(acc.shape[1], dtype=bool), "vector") for lane in range(WAVE)]
    return a_tile, b_tile, frags


def _verify_lane(intrinsic: Any, a_tile: _Masked, b_tile: _Masked, frag: _Masked, lane: int,
                 const: dict[str, Any]) -> None:
    verify = getattr(intrinsic, "__hc_verify__", None)
    if verify is None:
        return
    kwargs = {"lane": lane, **const}
    try:
        ok = verify(_CallSig(WorkItem, (_WaveGroup, a_tile, b_tile, frag), kwargs), None)
    except Exception as exc:  # noqa: BLE001 - the hook's failure is the verdict
        raise LaunchError(f"intrinsic {intrinsic.__name__!r} verify hook failed: {exc}") from exc
    if ok is False:
        raise LaunchError(f"intrinsic {intrinsic.__name__!r} verify hook returned False")


def fallback_wave(intrinsic: Any, a: np.ndarray, b: np.ndarray, acc: np.ndarray, *, dtype: str = "float16",
                  a_mask: np.ndarray | None = None, b_mask: np.ndarray | None = None, **const: Any) -> np.ndarray:
    """Every lane's result of the intrinsic's fallback body, (64, R) float32."""
    a_tile, b_tile, frags = _lane_args(a, b, acc, dtype, a_mask, b_mask)
    out = []
    for lane in range(WAVE):
        _verify_lane(intrinsic, a_tile, b_tile, frags[lane], lane, const)
        res = intrinsic(_WaveGroup, a_tile, b_tile, frags[lane], lane=lane, **const)
        if not isinstance(res, _Masked) or res.dtype != np.dtype(np.float32) or not res._mask.all():
            raise LaunchError(f"intrinsic {intrinsic.__name__!r} fallback did not return an active float32 vector")
        out.append(res._data)
    return np.stack(out)


def lowered_op(intrinsic: Any, a: np.ndarray, b: np.ndarray, acc: np.ndarray, *, dtype: str = "float16",
               a_mask: np.ndarray | None = None, b_mask: np.ndarray | None = None, **const: Any
               ) -> tuple[str, tuple[int, int, int]]:
    """(op name, (m, n, k)) the intrinsic's amdgpu-gfx950 lowering creates for
    this call; LaunchError if it has none or creates an op this library does
    not execute."""
    a_tile, b_tile, frags = _lane_args(a, b, acc, dtype, a_mask, b_mask)
    args = (_WaveGroup, a_tile, b_tile, frags[0])
    try:
        op = record_lowering(intrinsic, TARGET, args, {"lane": _Lane(), **const})
        shape = check_matrix_op(op, TARGET, intrinsic, args)
    except LoweringError as exc:
        raise LaunchError(str(exc)) from exc
    return op.name, shape


def run_wave(intrinsic: Any, a: np.ndarray, b: np.ndarray, acc: np.ndarray, *, dtype: str = "float16",
             a_mask: np.ndarray | None = None, b_mask: np.ndarray | None = None, **const: Any) -> np.ndarray:
    """Every lane's result of the op the intrinsic's amdgpu-gfx950 lowering
    creates, executed on the current GPU: (64, R) float32."""
    a_tile, b_tile, frags = _lane_args(a, b, acc, dtype, a_mask, b_mask)
    for lane in range(WAVE):
        _verify_lane(intrinsic, a_tile, b_tile, frags[lane], lane, const)
    _, (m, n, k) = lowered_op(intrinsic, a, b, acc, dtype=dtype, a_mask=a_mask, b_mask=b_mask, **const)
    regs = m * n // WAVE
    if np.shape(a) != (m, k) or np.shape(b) != (k, n) or np.shape(acc) != (WAVE, regs):
        raise LaunchError(f"the {m}x{n}x{k} instruction takes A {m}x{k}, B {k}x{n} and ({WAVE}, {regs}) "
                          f"accumulators, got {np.shape(a)}, {np.shape(b)} and {np.shape(acc)}")
    import torch

    dev = torch.device("cuda", torch.cuda.current_device())
    code = _native.HCG_F16 if dtype == "float16" else _native.HCG_BF16
    bits_a = np.ascontiguousarray(a, dtype=np.float16 if dtype == "float16" else np.uint16).view(np.int16)
    bits_b = np.ascontiguousarray(b, dtype=np.float16 if dtype == "float16" else np.uint16).view(np.int16)
    ta = torch.from_numpy(bits_a).to(dev)
    tb = torch.from_numpy(bits_b).to(dev)
    tam = torch.from_numpy(np.ascontiguousarray(a_tile._mask, dtype=np.uint8)).to(dev)
    tbm = torch.from_numpy(np.ascontiguousarray(b_tile._mask, dtype=np.uint8)).to(dev)
    t_in = torch.from_numpy(np.ascontiguousarray(acc, dtype=np.float32)).to(dev)
    t_out = torch.full((WAVE, regs), float("nan"), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    _native.mfma_step(code, m, n, k, ta.data_ptr(), tb.data_ptr(), tam.data_ptr(), tbm.data_ptr(), t_in.data_ptr(),
                      t_out.data_ptr(), stream)
    torch.cuda.synchronize(dev)
    return t_out.cpu().numpy()
