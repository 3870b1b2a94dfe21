"""Calling an intrinsic's registered lowering callback, and checking the op it
creates against the matrix-core instructions this library executes.

In the reference a lowering is ``cb(ctx, *args, **const_kwargs)``,
registered with ``@intrinsic.lower(target=...)`` (hc/core.py:282-307), that
overrides the fallback body on its target.  It builds the target op through
``ctx.builder.create(name, results=, operands=, attrs=, loc=)``,
``ctx.result_type(i)`` and ``ctx.loc`` and returns the op's result
(doc/langref.md:860-870 and 895-899; the gfx11 example,
examples/amdgpu_gfx11_wmma_matmul.py:200-228, creates one ``amdgpu.wmma`` op).
The reference only defines that contract (it lowers to MLIR and runs nothing).
Here ``ctx`` records the op instead of emitting IR, and the record decides
what runs:

* ``record_lowering`` calls a callback with a recording ``ctx`` and returns
  the one op it created (its name, result types, operands, attributes and
  location) -- or ``LoweringError`` if it created none or several, or does not
  return that op's result;
* ``check_matrix_op`` accepts the op only if its name is an instruction
  that a kernel of this library executes for the target, with attributes
  ``m``, ``n``, ``k``, ``arch`` and ``wave_size`` equal to that instruction's,
  one float32 vector result of ``m * n / wave_size`` lanes (the intrinsic's
  declared result type), and the call's accumulator as its last operand.

``amdgpu-gfx950`` ops run as themselves (``hcg_mfma_step``, and the same
instructions inside the GEMM kernels).  The reference's own
``amdgpu-gfx11`` WMMA op is accepted as the statement of a float32
accumulating 16x16x16 step; the gfx950 GEMM replaces the whole kernel that
uses it.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

from ..core import VectorTypeSpec

# target -> {op name: (m, n, k)}, and each target's (arch, wave_size).
TARGET_OPS: dict[str, dict[str, tuple[int, int, int]]] = {
    "amdgpu-gfx950": {
        "rocdl.mfma.f32.32x32x16": (32, 32, 16),  # v_mfma_f32_32x32x16_{f16,bf16}
        "rocdl.mfma.f32.16x16x32": (16, 16, 32),  # v_mfma_f32_16x16x32_{f16,bf16}
    },
    "amdgpu-gfx11": {
        "amdgpu.wmma": (16, 16, 16),  # v_wmma_f32_16x16x16_f16 (the reference's example)
    },
}
TARGET_ARCH: dict[str, tuple[str, int]] = {"amdgpu-gfx950": ("gfx950", 64), "amdgpu-gfx11": ("gfx11", 32)}
# Lowerings are looked up in this order: the device's own target first.
TARGET_ORDER = ("amdgpu-gfx950", "amdgpu-gfx11")


class LoweringError(Exception):
    """A lowering callback failed, or created an op this library does not run."""


@dataclass(frozen=True)
class Location:
    """``ctx.loc``: where the intrinsic is called."""

    file: str
    line: int

    def __str__(self) -> str:
        return f"{self.file}:{self.line}"


@dataclass(frozen=True)
class OpResult:
    op: RecordedOp
    index: int


@dataclass(eq=False)
class RecordedOp:
    """The op a lowering callback created through ``ctx.builder.create``."""

    name: str
    results: tuple[Any, ...]
    operands: tuple[Any, ...]
    attrs: dict[str, Any]
    loc: Any

    def result(self, index: int) -> OpResult:
        if not 0 <= index < len(self.results):
            raise IndexError(f"{self.name} has {len(self.results)} results, not {index + 1}")
        return OpResult(self, index)


@dataclass(eq=False)
class _Builder:
    ops: list[RecordedOp] = field(default_factory=list)

    def create(self, name: str, *, results: Any = (), operands: Any = (), attrs: Any = None,
               loc: Any = None) -> RecordedOp:
        if not isinstance(name, str) or not name:
            raise TypeError("builder.create: the op name must be a non-empty string")
        op = RecordedOp(name, tuple(results), tuple(operands), dict(attrs or {}), loc)
        self.ops.append(op)
        return op


class LoweringContext:
    """The ``ctx`` a lowering callback receives."""

    def __init__(self, intrinsic: Any, loc: Location | None) -> None:
        self.builder = _Builder()
        self.loc = loc
        self._results = tuple(getattr(intrinsic.__hc_intrinsic__, "result_types", ()) or ())
        self._name = intrinsic.__name__

    def result_type(self, index: int) -> Any:
        if not 0 <= index < len(self._results):
            raise IndexError(f"intrinsic {self._name!r} declares {len(self._results)} result types")
        return self._results[index]


def lowering_target(intrinsic: Any) -> str | None:
    """The first target of ``TARGET_ORDER`` the intrinsic has a lowering for."""
    lowerings = getattr(intrinsic, "__hc_lowerings__", None) or {}
    for target in TARGET_ORDER:
        if target in lowerings:
            return target
    return None


def record_lowering(intrinsic: Any, target: str, args: tuple[Any, ...], kwargs: dict[str, Any],
                    loc: Location | None = None) -> RecordedOp:
    """Calls ``intrinsic``'s ``target`` lowering with a recording ctx and the
    call's arguments; returns the op it created."""
    name = intrinsic.__name__
    callback = (getattr(intrinsic, "__hc_lowerings__", None) or {}).get(target)
    if callback is None:
        raise LoweringError(f"intrinsic {name!r} has no {target} lowering")
    ctx = LoweringContext(intrinsic, loc)
    try:
        out = callback(ctx, *args, **kwargs)
    except Exception as exc:  # noqa: BLE001 - the callback's failure is the verdict
        raise LoweringError(f"intrinsic {name!r}: its {target} lowering raised {type(exc).__name__}: {exc}") from exc
    ops = ctx.builder.ops
    if len(ops) != 1:
        raise LoweringError(f"intrinsic {name!r}: its {target} lowering creates {len(ops)} ops; "
                            "one matrix-core op is expected")
    op = ops[0]
    if not (isinstance(out, OpResult) and out.op is op and out.index == 0):
        raise LoweringError(f"intrinsic {name!r}: its {target} lowering does not return result 0 of the "
                            f"{op.name} op it creates")
    return op


def check_matrix_op(op: RecordedOp, target: str, intrinsic: Any, args: tuple[Any, ...]) -> tuple[int, int, int]:
    """(m, n, k) of ``op`` if it is an instruction this library executes for
    ``target`` as the intrinsic called with ``args`` would; else LoweringError."""
    name = intrinsic.__name__
    table = TARGET_OPS.get(target)
    if table is None:
        raise LoweringError(f"intrinsic {name!r}: this library executes no {target} ops")
    if op.name not in table:
        raise LoweringError(f"intrinsic {name!r}: its {target} lowering creates {op.name!r}, which no kernel of "
                            f"this library executes (it executes {', '.join(sorted(table))})")
    m, n, k = table[op.name]
    arch, wave = TARGET_ARCH[target]
    for key, want in (("m", m), ("n", n), ("k", k), ("arch", arch), ("wave_size", wave)):
        got = op.attrs.get(key)
        if got != want:
            raise LoweringError(f"intrinsic {name!r}: its {op.name} op declares {key}={got!r}, but that "
                                f"instruction has {key}={want!r}")
    want_type = VectorTypeSpec((m * n // wave,), "float32")
    if op.results != (want_type,):
        raise LoweringError(f"intrinsic {name!r}: its {op.name} op's results are {list(op.results)}, "
                            f"not one {want_type}")
    positional = list(args)
    if len(op.operands) != 3 or not all(any(o is a for a in positional) for o in op.operands):
        raise LoweringError(f"intrinsic {name!r}: its {op.name} op must take three of the call's arguments "
                            "(A, B, accumulator)")
    if not positional or op.operands[2] is not positional[-1]:
        raise LoweringError(f"intrinsic {name!r}: its {op.name} op must take the call's accumulator (its last "
                            "positional argument) as its last operand")
    return m, n, k
