"""Masked tile gather / scatter on gfx950.

The hc DSL's tile access (hc/simulator.py:296-358, 1304-1458;
doc/langref.md:530-596) over batches of tiles of a 2-D device tensor:

* ``tile_load(src, origins, (th, tw))`` is, per tile,
  ``group.load(src[r0:, c0:], shape=(th, tw))`` followed by
  ``with_inactive(fill)`` and ``.mask``: elements outside ``src`` are
  inactive and carry ``fill``; with ``mask=`` it is
  ``group.load(..., mask=m)`` (an element is active only if ``m`` is too);
* ``tile_store(dst, origins, tiles)`` is, per tile,
  ``group.store(dst[r0:, c0:], tile)``: only active elements inside ``dst``
  are written.

Coordinates outside ``src`` / ``dst`` (negative ones included) are out of
bounds.  The work runs in libhcg_gfx950.so (include/hcg_tile_ops.h) on the
tensor's device and current stream, asynchronously.
"""

from __future__ import annotations

from typing import Any

from .._errors import LaunchError
from . import _native

_ELEM_BYTES = (2, 4, 8)


def _torch():
    import torch

    return torch


def _origins(torch: Any, origins: Any, device: Any) -> Any:
    o = torch.as_tensor(origins, dtype=torch.int64, device=device)
    if o.ndim == 1 and o.numel() == 2:
        o = o.reshape(1, 2)
    if o.ndim != 2 or o.shape[1] != 2:
        raise LaunchError(f"origins must have shape (ntiles, 2), got {tuple(o.shape)}")
    return o.contiguous()


def _view(t: Any, what: str) -> tuple[int, int, int]:
    torch = _torch()
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise LaunchError(f"{what} must be a torch tensor on a GPU")
    if t.ndim != 2:
        raise LaunchError(f"{what} must be 2-D, got {t.ndim}-D")
    if t.element_size() not in _ELEM_BYTES:
        raise LaunchError(f"{what} element size must be 2, 4 or 8 bytes, got {t.element_size()}")
    rows, cols = t.shape
    if rows > 0 and cols > 1 and t.stride(1) != 1:
        raise LaunchError(f"{what} rows must be contiguous (stride(1) == 1)")
    ld = t.stride(0) if rows > 1 else cols
    return rows, cols, max(ld, cols)


def _mask(torch: Any, mask: Any, shape: tuple[int, int, int], device: Any) -> Any:
    if mask is None:
        return None
    m = torch.as_tensor(mask, device=device)
    if tuple(m.shape) != shape:
        raise LaunchError(f"mask shape {tuple(m.shape)} does not match the tiles {shape}")
    if m.dtype != torch.bool and m.dtype != torch.uint8:
        raise LaunchError(f"mask= expects a bool tensor, got {m.dtype}")
    return m.to(torch.uint8).contiguous()


def _fill_bits(torch: Any, fill: Any, dtype: Any) -> int:
    v = torch.tensor([fill], dtype=dtype)
    ints = {2: torch.int16, 4: torch.int32, 8: torch.int64}[v.element_size()]
    return int(v.view(ints).item()) & ((1 << (8 * v.element_size())) - 1)


def tile_load(src: Any, origins: Any, shape: tuple[int, int], *, mask: Any = None, fill: Any = 0) -> tuple[Any, Any]:
    """Gather tiles of ``shape`` from ``src`` at ``origins`` ((ntiles, 2)
    row/column pairs).  Returns ``(tiles, active)``: tiles of shape
    (ntiles, th, tw) in ``src``'s dtype, inactive elements set to ``fill``,
    and the bool activity of every element."""
    torch = _torch()
    rows, cols, ld = _view(src, "src")
    th, tw = (int(x) for x in shape)
    if th < 0 or tw < 0:
        raise LaunchError(f"tile shape must be non-negative, got {shape}")
    o = _origins(torch, origins, src.device)
    n = o.shape[0]
    m = _mask(torch, mask, (n, th, tw), src.device)
    out = torch.empty((n, th, tw), dtype=src.dtype, device=src.device)
    active = torch.empty((n, th, tw), dtype=torch.uint8, device=src.device)
    if out.numel() == 0:
        return out, active.view(torch.bool)
    with torch.cuda.device(src.device):
        stream = torch.cuda.current_stream(src.device).cuda_stream
        _native.tile_load(src.element_size(), src.data_ptr(), ld, rows, cols, o.data_ptr(), n, th, tw,
                          m.data_ptr() if m is not None else 0, _fill_bits(torch, fill, src.dtype),
                          out.data_ptr(), active.data_ptr(), stream)
    return out, active.view(torch.bool)


def tile_store(dst: Any, origins: Any, tiles: Any, *, mask: Any = None) -> None:
    """Scatter ``tiles`` ((ntiles, th, tw), ``dst``'s dtype) into ``dst`` at
    ``origins``: an element is written iff it lies inside ``dst`` and is
    active in ``mask`` (all active when None).  Tiles whose written elements
    overlap land in unspecified order."""
    torch = _torch()
    rows, cols, ld = _view(dst, "dst")
    if not isinstance(tiles, torch.Tensor) or tiles.ndim != 3:
        raise LaunchError("tiles must be a 3-D torch tensor (ntiles, th, tw)")
    if tiles.dtype != dst.dtype:
        raise LaunchError(f"tiles dtype {tiles.dtype} does not match dst dtype {dst.dtype}")
    if tiles.device != dst.device:
        raise LaunchError("tiles and dst must live on the same device")
    n, th, tw = tiles.shape
    o = _origins(torch, origins, dst.device)
    if o.shape[0] != n:
        raise LaunchError(f"{o.shape[0]} origins for {n} tiles")
    m = _mask(torch, mask, (n, th, tw), dst.device)
    t = tiles.contiguous()
    if t.numel() == 0 or rows == 0 or cols == 0:
        return
    with torch.cuda.device(dst.device):
        stream = torch.cuda.current_stream(dst.device).cuda_stream
        _native.tile_store(dst.element_size(), dst.data_ptr(), ld, rows, cols, o.data_ptr(), n, th, tw,
                           t.data_ptr(), m.data_ptr() if m is not None else 0, stream)
