"""``hc.compile(fn)`` -> ``CompiledKernel`` whose call launches on gfx950.

The reference's ``compile`` runs the MLIR frontend pipeline and returns a
handle whose ``__call__`` raises NotImplementedError (hc/_compile.py:57-62,
71-150); the documented intent is that calling it launches the compiled
kernel (doc/lowering.md:776-788).  Here the MLIR pipeline is out of scope and
the handle launches through the gfx950 target: ``compile`` checks that a
gfx950 lowering exists for the kernel, and each call performs the usual
binding and validation.  ``symbols`` pins symbol values; a call whose buffers
bind a pinned symbol to another value raises ``LaunchError``.
"""

from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass, field
from typing import Any

from ._errors import LaunchError
from ._launch import kernel_metadata, prepare_launch
from .symbols import Symbol, sym_of


@dataclass
class CompiledKernel:
    kernel: Any
    symbols: dict[Symbol, int] = field(default_factory=dict)
    target: Any = None
    hc_ir_text: str | None = None
    pipeline_diagnostics: tuple[str, ...] = ()

    def __call__(self, *args: Any, **kwargs: Any) -> None:
        from . import gfx950

        target = self.target or gfx950.Gfx950Target()
        prepared = prepare_launch(self.kernel, args, kwargs, target)
        for symbol, value in self.symbols.items():
            bound = prepared.env.get(symbol)
            if bound is not None and bound != value:
                raise LaunchError(
                    f"{symbol} is compiled as {value} but the arguments bind {bound}"
                )
        lowering = gfx950.find_lowering(self.kernel)
        if prepared.is_empty:
            return
        lowering(prepared, target)


def compile(  # noqa: A001 - reference name
    kernel_fn: Any,
    symbols: Mapping[Any, int] | None = None,
    *,
    schedule: Any = None,
    target: Any = None,
) -> CompiledKernel:
    kernel_metadata(kernel_fn)
    if schedule is not None:
        raise LaunchError("transform schedules are not supported by the gfx950 backend")
    from . import gfx950

    gfx950.find_lowering(kernel_fn)
    pinned: dict[Symbol, int] = {}
    for key, value in (symbols or {}).items():
        symbol = sym_of(key) if isinstance(key, str) else key
        if not isinstance(symbol, Symbol):
            raise LaunchError(f"symbols keys must be symbols or names, got {key!r}")
        pinned[symbol] = int(value)
    return CompiledKernel(kernel=kernel_fn, symbols=pinned, target=target)
