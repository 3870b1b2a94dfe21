"""Kernel-definition surface of the hc DSL: decorators, buffer and type specs,
scope objects and the intrinsic hook registry.

Same names, signatures and attached metadata as the reference's
hc/core.py so that kernel modules written against it import and launch
unchanged:

* ``@kernel(work_shape=, group_shape=, subgroup_size=, literals=)`` attaches
  ``fn.__hc_kernel__ = KernelMetadata(...)`` and returns the same function
  (hc/core.py:310-334, metadata :144-149);
* ``@kernel.func(scope=)`` attaches ``__hc_func__`` (:336-352);
* ``@kernel.intrinsic(scope, effects, const_attrs, operand_types,
  result_types)`` attaches ``__hc_intrinsic__`` plus the hook registry
  ``.lower(target=)``, ``.verify``, ``.infer`` and ``__hc_has_fallback__``
  (:354-389, hooks :282-307);
* ``Buffer[M, K, np.float16]`` -> ``BufferSpec(dims, dtype_name)`` (:17-27,
  :68-92).

Addition for gfx950: ``bfloat16`` is a dtype marker accepted in ``Buffer[...]``
and the type specs (NumPy has no bfloat16; the reference's element types are
NumPy dtypes only).
"""

from __future__ import annotations

import ast
import functools
import inspect
import textwrap
from collections.abc import Callable, Sequence
from dataclasses import dataclass, field
from typing import Any


class _BFloat16:
    """Element-type marker for bfloat16 (no NumPy dtype exists for it)."""

    name = "bfloat16"

    def __repr__(self) -> str:
        return "bfloat16"


bfloat16 = _BFloat16()


def _dtype_name(value: Any) -> str:
    if value is bfloat16 or value == "bfloat16":
        return "bfloat16"
    import numpy as np

    return str(np.dtype(value).name)


def _buffer_dtype_name(value: Any) -> str | None:
    """Trailing Buffer[...] item -> dtype name, or None if it is a dimension."""
    import numpy as np

    if value is bfloat16:
        return "bfloat16"
    if isinstance(value, np.dtype):
        return str(value.name)
    if isinstance(value, type) and issubclass(value, np.generic):
        return str(np.dtype(value).name)
    return None


@dataclass(frozen=True)
class BufferSpec:
    dimensions: tuple[Any, ...]
    dtype: str | None = None

    def __repr__(self) -> str:
        parts = [str(d) for d in self.dimensions]
        if self.dtype is not None:
            parts.append(self.dtype)
        return "Buffer[" + ", ".join(parts) + "]"


class Buffer:
    """``Buffer[dims..., dtype]`` annotation factory."""

    def __class_getitem__(cls, item: Any) -> BufferSpec:
        items = item if isinstance(item, tuple) else (item,)
        dtype = _buffer_dtype_name(items[-1]) if len(items) >= 2 else None
        dims = items[:-1] if dtype is not None else items
        return BufferSpec(tuple(dims), dtype=dtype)


@dataclass(frozen=True)
class TensorTypeSpec:
    dimensions: tuple[Any, ...]
    dtype: str


@dataclass(frozen=True)
class VectorTypeSpec:
    dimensions: tuple[Any, ...]
    dtype: str


@dataclass(frozen=True)
class IdxTypeSpec:
    expr: Any = None


@dataclass(frozen=True)
class UndefTypeSpec:
    pass


def tensor_type(shape: Sequence[Any], dtype: Any) -> TensorTypeSpec:
    return TensorTypeSpec(tuple(shape), _dtype_name(dtype))


def vector_type(shape: Sequence[Any], dtype: Any) -> VectorTypeSpec:
    return VectorTypeSpec(tuple(shape), _dtype_name(dtype))


def idx_type(expr: Any = None) -> IdxTypeSpec:
    return IdxTypeSpec(expr)


def undef_type() -> UndefTypeSpec:
    return UndefTypeSpec()


@dataclass(frozen=True)
class Scope:
    name: str

    def __str__(self) -> str:
        return self.name

    __repr__ = __str__


WorkGroup = Scope("WorkGroup")


@dataclass(frozen=True)
class Result:
    type: Any
    mask: Any = None
    layout: Any = None


@dataclass(frozen=True)
class IndexMap:
    params: Callable[..., Any] | None
    storage_size: Callable[..., Any]
    offset: Callable[..., Any]


def index_map(
    *,
    params: Callable[..., Any] | None = None,
    storage_size: Callable[..., Any],
    offset: Callable[..., Any],
) -> IndexMap:
    return IndexMap(params=params, storage_size=storage_size, offset=offset)


def as_layout(value: Any, layout: Any = None) -> Any:
    method = getattr(value, "as_layout", None)
    if method is None:
        raise TypeError("as_layout() expects a layout-aware value")
    return method(layout)


@dataclass(frozen=True)
class KernelMetadata:
    work_shape: Any = None
    group_shape: Any = None
    subgroup_size: Any = None
    literals: frozenset[Any] = field(default_factory=frozenset)


@dataclass(frozen=True)
class FuncMetadata:
    scope: Any = None


@dataclass(frozen=True)
class IntrinsicMetadata:
    scope: Any = None
    effects: Any = None
    const_attrs: frozenset[str] = field(default_factory=frozenset)
    operand_types: tuple[Any, ...] | None = None
    result_types: tuple[Any, ...] = ()


def _body_is_placeholder(fn: Callable[..., Any]) -> bool | None:
    """True if the body is empty, ``pass`` or ``...`` (after a docstring);
    None when the source cannot be read."""
    try:
        source = textwrap.dedent(inspect.getsource(fn))
        tree = ast.parse(source)
    except (OSError, TypeError, SyntaxError):
        return None
    node = tree.body[0] if tree.body else None
    if not isinstance(node, (ast.FunctionDef, ast.AsyncFunctionDef)):
        return None
    body = list(node.body)
    if (
        body
        and isinstance(body[0], ast.Expr)
        and isinstance(body[0].value, ast.Constant)
        and isinstance(body[0].value.value, str)
    ):
        body = body[1:]
    if not body:
        return True
    if len(body) > 1:
        return False
    stmt = body[0]
    if isinstance(stmt, ast.Pass):
        return True
    return isinstance(stmt, ast.Expr) and isinstance(stmt.value, ast.Constant) and stmt.value.value is Ellipsis


def _has_fallback(fn: Callable[..., Any]) -> bool:
    placeholder = _body_is_placeholder(fn)
    if placeholder is None:
        # Without source, count anything beyond "return None" as a body.
        code = fn.__code__
        return len(code.co_code) > 4 or code.co_consts not in ((None,), ())
    return not placeholder


class _IntrinsicHooks:
    """The per-intrinsic hook surface of hc/core.py:282-307, bound to one
    intrinsic function: ``fn.lower(target=...)`` registers a lowering in
    ``fn.__hc_lowerings__`` (target name -> callback), ``fn.verify`` and
    ``fn.infer`` set ``fn.__hc_verify__`` and ``fn.__hc_infer__``; each
    decorator returns the callback unchanged."""

    def __init__(self, fn: Any) -> None:
        self._fn = fn
        fn.__hc_lowerings__ = {}
        fn.__hc_verify__ = None
        fn.__hc_infer__ = None
        fn.__hc_has_fallback__ = _has_fallback(fn)

    def lower(self, *, target: str) -> Callable[[Callable[..., Any]], Callable[..., Any]]:
        return functools.partial(self._record_lowering, target)

    def _record_lowering(self, target: str, cb: Callable[..., Any]) -> Callable[..., Any]:
        self._fn.__hc_lowerings__[target] = cb
        return cb

    def verify(self, cb: Callable[..., Any]) -> Callable[..., Any]:
        self._fn.__hc_verify__ = cb
        return cb

    def infer(self, cb: Callable[..., Any]) -> Callable[..., Any]:
        self._fn.__hc_infer__ = cb
        return cb


def _attach_intrinsic_hooks(fn: Any) -> Any:
    hooks = _IntrinsicHooks(fn)
    fn.lower, fn.verify, fn.infer = hooks.lower, hooks.verify, hooks.infer
    return fn


class _KernelNamespace:
    def __call__(
        self,
        fn: Callable[..., Any] | None = None,
        *,
        work_shape: Any = None,
        group_shape: Any = None,
        subgroup_size: Any = None,
        literals: set[Any] | frozenset[Any] | None = None,
    ) -> Any:
        metadata = KernelMetadata(
            work_shape=work_shape,
            group_shape=group_shape,
            subgroup_size=subgroup_size,
            literals=frozenset(literals or ()),
        )

        def decorate(target: Any) -> Any:
            target.__hc_kernel__ = metadata
            return target

        return decorate if fn is None else decorate(fn)

    def func(self, fn: Callable[..., Any] | None = None, *, scope: Any = None) -> Any:
        metadata = FuncMetadata(scope=scope)

        def decorate(target: Any) -> Any:
            target.__hc_func__ = metadata
            return target

        return decorate if fn is None else decorate(fn)

    def intrinsic(
        self,
        fn: Callable[..., Any] | None = None,
        *,
        scope: Any = None,
        effects: Any = None,
        const_attrs: set[str] | frozenset[str] | None = None,
        operand_types: Sequence[Any] | None = None,
        result_types: Sequence[Any] | Any = (),
    ) -> Any:
        if result_types is None:
            results: tuple[Any, ...] = ()
        elif isinstance(result_types, Sequence) and not isinstance(result_types, (str, bytes)):
            results = tuple(result_types)
        else:
            results = (result_types,)
        metadata = IntrinsicMetadata(
            scope=scope,
            effects=effects,
            const_attrs=frozenset(const_attrs or ()),
            operand_types=None if operand_types is None else tuple(operand_types),
            result_types=results,
        )

        def decorate(target: Any) -> Any:
            target.__hc_intrinsic__ = metadata
            return _attach_intrinsic_hooks(target)

        return decorate if fn is None else decorate(fn)


kernel = _KernelNamespace()


class CurrentGroup:
    """Workgroup handle passed as a kernel's first argument.  Runtime backends
    supply the behaviour; on gfx950 kernels are lowered as a whole, so these
    host stubs are never executed by a launch."""

    def __init__(
        self,
        *,
        group_id: tuple[int, ...] = (),
        shape: tuple[int, ...] = (),
        work_shape: tuple[int, ...] = (),
        work_offset: tuple[int, ...] = (),
    ) -> None:
        self.group_id = group_id
        self.shape = shape
        self.work_shape = work_shape
        self.work_offset = work_offset

    @property
    def size(self) -> int:
        total = 1
        for dim in self.shape:
            total *= dim
        return total

    def subgroups(self, fn: Callable[..., Any]) -> Callable[..., Any]:
        return fn

    def workitems(self, fn: Callable[..., Any]) -> Callable[..., Any]:
        return fn


class SubGroup:
    """A subgroup's view inside a kernel (``subgroup_id()``, ``size()``); only a
    runtime gives the methods meaning."""


class WorkItem:
    """A work item's view inside a kernel (``global_id()``, ``local_id()``);
    only a runtime gives the methods meaning."""


def _outside_launch(owner: str, name: str) -> Callable[..., Any]:
    def method(self: Any, *args: Any, **kwargs: Any) -> Any:
        raise NotImplementedError(
            f"{owner}.{name}() means something only while a kernel runs: launch it with "
            "hc.simulator.launch, hc.gfx950.launch or hc.compile(kernel)(...)")

    method.__name__ = method.__qualname__ = name
    return method


for _owner, _cls, _names in (
    ("group", CurrentGroup, ("barrier", "load", "vload", "store", "empty", "zeros", "ones", "full", "vzeros",
                             "vones", "vfull")),
    ("subgroup", SubGroup, ("subgroup_id", "size")),
    ("workitem", WorkItem, ("global_id", "local_id")),
):
    for _name in _names:
        setattr(_cls, _name, _outside_launch(_owner, _name))
del _owner, _cls, _names, _name
