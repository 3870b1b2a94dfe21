"""hc kernel DSL surface with a gfx950 (MI355X) backend.

Exports the reference's public names (hc/__init__.py:11-66) so kernel
modules written against ``hc`` import unchanged; ``hc.simulator`` and
``hc.symbols`` load lazily as in the reference (hc/__init__.py:68-95), and
``hc.gfx950`` holds the GPU target.
"""

from __future__ import annotations

import importlib
from typing import Any

from ._compile import CompiledKernel, compile
from ._errors import BackendError, LaunchError, SimulatorError
from .core import (
    Buffer,
    BufferSpec,
    CurrentGroup,
    IdxTypeSpec,
    IndexMap,
    Result,
    Scope,
    SubGroup,
    TensorTypeSpec,
    UndefTypeSpec,
    VectorTypeSpec,
    WorkGroup,
    WorkItem,
    as_layout,
    bfloat16,
    idx_type,
    index_map,
    kernel,
    tensor_type,
    undef_type,
    vector_type,
)
from .symbols import Symbol, sym

__all__ = [
    "BackendError",
    "Buffer",
    "BufferSpec",
    "CompiledKernel",
    "CurrentGroup",
    "IdxTypeSpec",
    "IndexMap",
    "LaunchError",
    "Result",
    "Scope",
    "SimulatorError",
    "SubGroup",
    "Symbol",
    "TensorTypeSpec",
    "UndefTypeSpec",
    "VectorTypeSpec",
    "WorkGroup",
    "WorkItem",
    "as_layout",
    "bfloat16",
    "compile",
    "gfx950",
    "idx_type",
    "index_map",
    "kernel",
    "simulator",
    "sym",
    "symbols",
    "tensor_type",
    "undef_type",
    "vector_type",
]

_LAZY = {"simulator": ".simulator", "symbols": ".symbols", "gfx950": ".gfx950"}


def __getattr__(name: str) -> Any:
    if name in _LAZY:
        return importlib.import_module(_LAZY[name], __name__)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


def __dir__() -> list[str]:
    return sorted(__all__)
