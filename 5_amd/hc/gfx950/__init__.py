"""gfx950 (MI355X) launch target for hc kernels.

``launch(fn, *args, target=Gfx950Target())`` keeps the reference launch
contract (hc/simulator.py:165-186): the same argument binding and geometry
validation (see ``hc._launch``), ``LaunchError`` before any execution, and a
zero-size launch is a no-op.  It then runs the kernel as a whole on the GPU
through the C ABI of libhcg_gfx950.so (include/hcg_gemm.h) instead of
interpreting it workgroup by workgroup.

Kernels are lowered as a whole, not intrinsic by intrinsic: the wave64 MFMA
design replaces the reference's per-lane wave32 WMMA fragment contract
(examples/amdgpu_gfx11_wmma_matmul.py:18-31), so no per-intrinsic mapping
exists.  A kernel runs on gfx950 when

* its body is the tiled contraction of
  examples/amdgpu_gfx11_wmma_matmul.py:306-326 (any tile extents), checked
  statement by statement and by a recorded CPU run of a small ragged launch
  through the kernel's own helpers and intrinsic fallbacks, whose intrinsic
  carries a lowering for an amdgpu target (see ``_contract``) -- the
  reference's ``tiled_gfx11_wmma_matmul`` and this package's
  ``tiled_gfx950_mfma_matmul`` both are; or
* a lowering callable was registered for it with :func:`register_kernel`.

Anything else raises ``LaunchError`` naming the kernel and the reason; the
kernel's name plays no part.
"""

from __future__ import annotations

import functools
import os
from collections.abc import Callable
from dataclasses import dataclass
from typing import Any

import numpy as np

from .._errors import BackendError, LaunchError
from .._launch import PreparedLaunch, buffer_dtype_name, prepare_launch
from . import _native
from ._contract import TARGET_NAME, Contraction, gemm_signature, recognise

_DTYPE_CODES = {"float16": _native.HCG_F16, "bfloat16": _native.HCG_BF16}
_TORCH_DTYPE_CODES: dict[Any, int] = {}


@dataclass(frozen=True)
class Gfx950Target:
    """Launch policy for gfx950 (the counterpart of ``SimulatorTarget``,
    hc/simulator.py:60-75).

    device: GPU index for host (numpy) buffers; device tensors run where they
        live.  None = the current device.
    algo: "auto" (by shape), "tiled", "skinny" (M <= 128, any layout
        whose B holds at least 8 elements) or "narrow" (N <= 64, any
        layout).
    max_group_size: HIP's workgroup limit, checked like the simulator's.
    """

    device: int | None = None
    algo: str = "auto"
    max_group_size: int | None = 1024
    name: str = TARGET_NAME

    def choose_group_shape(self, work_shape: tuple[int, ...], subgroup_size: int | None) -> tuple[int, ...]:
        base = tuple(max(1, d) for d in work_shape)
        if not base or subgroup_size is None:
            return base
        return (-(-base[0] // subgroup_size) * subgroup_size, *base[1:])


@functools.lru_cache(maxsize=1)
def device_available() -> bool:
    """True when the library is built and a gfx950 GPU is visible: then a
    launch with ``target=None`` runs here."""
    if not os.path.exists(_native.LIB_PATH):
        return False
    try:
        import torch
    except ImportError:
        return False
    if not torch.cuda.is_available():
        return False
    try:
        index = torch.cuda.current_device()
        arch = getattr(torch.cuda.get_device_properties(index), "gcnArchName", "") or ""
    except (RuntimeError, AssertionError):
        return False
    return arch.split(":")[0] == "gfx950"


# --------------------------------------------------------------------------
# Kernel lowering registry
# --------------------------------------------------------------------------

Lowering = Callable[[PreparedLaunch, Gfx950Target], None]

_LOWERINGS: dict[Any, Lowering] = {}


def _contraction_lowering(contraction: Contraction) -> Lowering:
    def lower(prepared: PreparedLaunch, target: Gfx950Target) -> None:
        args = prepared.bound.arguments
        gemm(args[contraction.a], args[contraction.b], out=args[contraction.c], algo=target.algo,
             device=target.device)

    lower.contraction = contraction  # type: ignore[attr-defined]
    return lower


def register_kernel(fn: Any, lowering: Lowering | str = "gemm") -> Any:
    """Register a gfx950 lowering for kernel ``fn``.

    ``"gemm"`` checks now that ``fn`` is the tiled contraction (the same
    check a launch makes, raising ``LaunchError`` if it is not); a callable
    ``lowering(prepared, target)`` replaces the whole launch of ``fn`` and is
    the caller's responsibility."""
    if not hasattr(fn, "__hc_kernel__"):
        raise LaunchError("register_kernel() expects a function decorated with @kernel")
    if lowering == "gemm":
        recognise(fn, Gfx950Target())
        return fn
    if not callable(lowering):
        raise TypeError("lowering must be 'gemm' or a callable")
    _LOWERINGS[fn] = lowering
    return fn


def find_lowering(fn: Any) -> Lowering:
    """The registered lowering of ``fn``, else the GEMM if ``fn`` is the
    tiled contraction; ``LaunchError`` otherwise."""
    lowering = _LOWERINGS.get(fn)
    if lowering is not None:
        return lowering
    if not hasattr(fn, "__hc_kernel__"):
        raise LaunchError("launch() expects a function decorated with @kernel")
    return _contraction_lowering(recognise(fn, Gfx950Target()))


def launch(fn: Any, *args: Any, target: Gfx950Target | None = None, **kwargs: Any) -> None:
    """Launch an hc kernel on gfx950 (contract of hc/simulator.py:165-186)."""
    runtime_target = Gfx950Target() if target is None else target
    prepared = prepare_launch(fn, args, kwargs, runtime_target)
    lowering = find_lowering(fn)
    if prepared.is_empty:
        return
    lowering(prepared, runtime_target)


run = launch


# --------------------------------------------------------------------------
# GEMM entry for numpy arrays and torch tensors
# --------------------------------------------------------------------------


_TORCH: Any = None


def _torch():
    global _TORCH
    if _TORCH is None:
        try:
            import torch
        except ImportError as exc:  # pragma: no cover - torch is present on the targets
            raise BackendError("the gfx950 backend needs PyTorch-ROCm for device memory") from exc
        _TORCH = torch
    return _TORCH


def _check_shapes(a: Any, b: Any, c: Any | None) -> tuple[int, int, int]:
    sa, sb = a.shape, b.shape
    if len(sa) != 2 or len(sb) != 2:
        raise LaunchError("A and B must be rank-2 matrices")
    m, k = sa
    k2, n = sb
    if k != k2:
        raise LaunchError("A.shape[1] must match B.shape[0]")
    if c is not None:
        sc = c.shape
        if len(sc) != 2 or sc[0] != m or sc[1] != n:
            raise LaunchError(f"C shape {tuple(sc)} does not match ({m}, {n})")
    return int(m), int(n), int(k)


def _dtype_code(a: Any, b: Any) -> int:
    da, db = buffer_dtype_name(a), buffer_dtype_name(b)
    if da != db or da not in _DTYPE_CODES:
        raise LaunchError(f"A and B must both be float16 or both bfloat16, got {da} and {db}")
    return _DTYPE_CODES[da]


def gemm(a: Any, b: Any, out: Any | None = None, *, algo: str = "auto", device: int | None = None) -> Any:
    """C = A @ B on gfx950 with float32 accumulation and output.

    Device tensors (torch, on a GPU) run in place on the current stream of
    their device, asynchronously.  numpy arrays are copied to the device,
    computed, and copied back into ``out`` (created if None); the call then
    returns after the result is on the host.

    ``algo``: "auto" (the library picks: the narrow streaming kernel for
    N <= 64; the streaming kernel for M <= 64, and for M <= 128 when the
    tiled kernel cannot read B in place; otherwise the LDS-tiled kernel
    with a modelled tile shape and K split, with up to 128 rows or 64
    columns past a multiple of 256 peeled off to a streaming kernel when
    that saves a round of tiles.  Operands are read in place at any row
    alignment; one whose last 16-byte piece cannot be read safely is
    repacked, or goes through registers),
    "tiled", "skinny", "narrow", "generic", or a fixed tile shape
    "tiled_256x256", "tiled_256x192", "tiled_128x256", "tiled_128x128",
    "tiled_256x64" (never split along K).
    """
    algo_code = _native.ALGOS.get(algo)
    if algo_code is None:
        raise LaunchError(f"unknown algo {algo!r}; expected one of {sorted(_native.ALGOS)}")
    torch_mod = _torch()
    tensor = torch_mod.Tensor
    if isinstance(a, tensor) and isinstance(b, tensor) and (out is None or isinstance(out, tensor)):
        return _gemm_torch(torch_mod, a, b, out, algo_code)
    if isinstance(a, np.ndarray) and isinstance(b, np.ndarray) and (out is None or isinstance(out, np.ndarray)):
        return _gemm_numpy(torch_mod, a, b, out, algo_code, device)
    raise LaunchError("A, B and C must all be numpy arrays or all be torch tensors")


def _gemm_numpy(torch: Any, a: np.ndarray, b: np.ndarray, out: np.ndarray | None, algo: int, device: int | None) -> np.ndarray:
    m, n, k = _check_shapes(a, b, out)
    if out is not None and out.dtype != np.float32:
        raise LaunchError(f"C dtype expected float32, got {out.dtype.name}")
    dtype = _dtype_code(a, b)
    if out is None:
        out = np.empty((m, n), dtype=np.float32)
    if m == 0 or n == 0:
        return out
    dev = torch.device("cuda", torch.cuda.current_device() if device is None else device)
    with torch.cuda.device(dev):
        ta = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        tb = torch.from_numpy(np.ascontiguousarray(b)).to(dev)
        tc = torch.empty((m, n), dtype=torch.float32, device=dev)
        stream = torch.cuda.current_stream(dev).cuda_stream
        _native.gemm(algo, dtype, ta.data_ptr(), max(k, 1), tb.data_ptr(), n, tc.data_ptr(), n, m, n, k, stream)
        out[...] = tc.cpu().numpy()
    return out


def _torch_dtype_code(torch: Any, a: Any, b: Any) -> int:
    if not _TORCH_DTYPE_CODES:
        _TORCH_DTYPE_CODES.update({torch.float16: _native.HCG_F16, torch.bfloat16: _native.HCG_BF16})
    code = _TORCH_DTYPE_CODES.get(a.dtype)
    if code is None or b.dtype != a.dtype:
        return _dtype_code(a, b)  # raises, naming both dtypes
    return code


_RAW_STREAM: Any = None
_CUR_DEVICE: Any = None


def _current_stream(torch: Any, index: int) -> int:
    """Raw handle of the current torch stream of device ``index``.

    ``torch._C._cuda_getCurrentRawStream`` returns it without building a
    ``torch.cuda.Stream`` object (a few microseconds per call); the public
    route is kept for a torch build that lacks it."""
    global _RAW_STREAM
    if _RAW_STREAM is None:
        _RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None) or (
            lambda i: torch.cuda.current_stream(i).cuda_stream)
    return _RAW_STREAM(index)


def _current_device(torch: Any) -> int:
    """Index of the current device (CUDA is initialised: a tensor lives
    there).  torch._C._cuda_getDevice skips torch.cuda.current_device()'s
    lazy-initialisation check."""
    global _CUR_DEVICE
    if _CUR_DEVICE is None:
        _CUR_DEVICE = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device
    return _CUR_DEVICE()


_FAST: Any = None  # _hcg_torch.gemm once loaded; False when the binding is not built


def _fast_gemm() -> Any:
    """The compiled device-tensor binding (_hcg_torch, built beside the
    library): the common case's checks and launch in C++, without the
    Python attribute reads below.  It runs the same library; where it is
    not built, the ctypes path below runs instead."""
    global _FAST
    if _FAST is None:
        _native.load()  # the library first: the binding links against it
        try:
            from . import _hcg_torch
        except ImportError as exc:
            # Calls still run (through ctypes), at about 1.5 us more host
            # time each; say so once rather than slow down silently.
            import warnings

            warnings.warn(f"hc.gfx950: the compiled device-tensor binding did not load ({exc}); "
                          "calls on torch tensors go through ctypes", RuntimeWarning, stacklevel=3)
            _FAST = False
        else:
            _FAST = _hcg_torch.gemm
    return _FAST


def _gemm_torch(torch: Any, a: Any, b: Any, out: Any | None, algo: int) -> Any:
    if out is not None:
        fast = _FAST if _FAST is not None else _fast_gemm()
        if fast:
            rc = fast(a, b, out, algo)  # -1: a case the binding leaves to the path below
            if rc == 0:
                return out
            if rc > 0:
                _native.check(_native.lib(), rc, "hcg_gemm")
    # (A call costs a few microseconds of host time, about as long as a
    # small GEMM's kernel: each tensor attribute is read once.)
    m, n, k = _check_shapes(a, b, out)
    index = a.get_device()  # -1 on the CPU
    ib, io = b.get_device(), (index if out is None else out.get_device())
    if index < 0 or ib < 0 or io < 0:
        raise LaunchError("torch tensors must live on a GPU")
    if ib != index or io != index:
        raise LaunchError("A, B and C must live on the same device")
    dta = a.dtype
    dtype = _TORCH_DTYPE_CODES.get(dta) if _TORCH_DTYPE_CODES else None
    if dtype is None or b.dtype is not dta:
        dtype = _torch_dtype_code(torch, a, b)
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=a.device)
    elif out.dtype != torch.float32:
        raise LaunchError(f"C dtype expected float32, got {str(out.dtype).replace('torch.', '')}")
    if m == 0 or n == 0:
        return out
    sa, sb, so = a.stride(), b.stride(), out.stride()
    if k > 0 and (sa[1] != 1 or (m > 1 and sa[0] < k)):
        a = a.contiguous()
        sa = a.stride()
    if k > 0 and (sb[1] != 1 or (k > 1 and sb[0] < n)):
        b = b.contiguous()
        sb = b.stride()
    direct = (so[1] == 1 or n == 1) and (m == 1 or so[0] >= n)
    target = out if direct else torch.empty((m, n), dtype=torch.float32, device=a.device)
    st = so if direct else target.stride()
    # Row strides as the C ABI reads them: a one-row matrix's stride is
    # unused, so report the smallest legal one.
    lda = max(sa[0], k) if m > 1 else max(k, 1)
    ldb = max(sb[0], n) if k > 1 else max(n, 1)
    ldc = max(st[0], n) if m > 1 else max(n, 1)
    if _current_device(torch) == index:
        lib = _native.lib()
        rc = lib.hcg_gemm_algo(algo, dtype, a.data_ptr(), lda, b.data_ptr(), ldb, target.data_ptr(), ldc, m, n, k,
                               _current_stream(torch, index) or None)
        if rc:
            _native.check(lib, rc, "hcg_gemm")
    else:
        with torch.cuda.device(index):
            _native.gemm(algo, dtype, a.data_ptr(), lda, b.data_ptr(), ldb, target.data_ptr(), ldc, m, n, k,
                         _current_stream(torch, index))
    if target is not out:
        out.copy_(target)
    return out


from .tiles import tile_load, tile_store  # noqa: E402  (masked tile gather / scatter)


def library_path() -> str:
    return _native.LIB_PATH


def library_available() -> bool:
    return os.path.exists(_native.LIB_PATH)


__all__ = [
    "Gfx950Target",
    "TARGET_NAME",
    "device_available",
    "find_lowering",
    "gemm",
    "launch",
    "library_available",
    "library_path",
    "register_kernel",
    "run",
    "tile_load",
    "tile_store",
]
