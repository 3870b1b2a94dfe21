"""Launch binding and geometry validation shared by every hc target.

Follows the reference's pre-execution phase (hc/simulator.py:189-229):
kernel metadata lookup (:657-661), binding the launch arguments without the
group parameter (:664-672), binding Buffer extents to symbols with conflict
detection (:675-683, :752-791), resolving ``work_shape``/``group_shape``/
``subgroup_size`` (:797-855) and validating the geometry (:858-900).  Symbol
errors surface as ``LaunchError`` (:227-228).

Buffers may be ``numpy.ndarray`` (as in the reference) or ``torch.Tensor``
(device buffers that a gfx950 launch uses in place).
"""

from __future__ import annotations

import inspect
from dataclasses import dataclass
from typing import Any, get_args, get_origin

from ._errors import LaunchError
from .core import BufferSpec, KernelMetadata
from .symbols import Bindings, Env, Expr, Symbol, SymbolError, sym


@dataclass(frozen=True)
class PreparedLaunch:
    fn: Any
    bound: inspect.BoundArguments
    env: Env
    literal_names: frozenset[str]
    work_shape: tuple[int, ...]
    group_shape: tuple[int, ...]
    subgroup_size: int | None
    buffer_params: tuple[str, ...]

    @property
    def is_empty(self) -> bool:
        return any(dim == 0 for dim in self.work_shape)


def buffer_dtype_name(value: Any) -> str | None:
    """dtype name of a numpy array or torch tensor, else None."""
    import numpy as np

    if isinstance(value, np.ndarray):
        return str(value.dtype.name)
    torch = _torch_if_loaded()
    if torch is not None and isinstance(value, torch.Tensor):
        return str(value.dtype).replace("torch.", "")
    return None


def _torch_if_loaded() -> Any:
    import sys

    return sys.modules.get("torch")


def is_buffer(value: Any) -> bool:
    return buffer_dtype_name(value) is not None


def kernel_metadata(fn: Any) -> KernelMetadata:
    metadata = getattr(fn, "__hc_kernel__", None)
    if metadata is None:
        raise LaunchError("launch() expects a function decorated with @kernel")
    return metadata


def _bind_arguments(fn: Any, args: tuple[Any, ...], kwargs: dict[str, Any]) -> inspect.BoundArguments:
    params = list(inspect.signature(fn).parameters.values())
    if not params:
        raise LaunchError("kernel must accept a CurrentGroup parameter")
    try:
        return inspect.Signature(params[1:]).bind(*args, **kwargs)
    except TypeError as exc:
        raise LaunchError(f"cannot bind launch arguments: {exc}") from exc


class _SymbolFallback(dict):
    """Evaluation namespace for string annotations: the kernel's closure
    variables, then its globals, and any other capitalised name becomes the
    symbol of that name (``Buffer["M", "K"]`` style annotations)."""

    def __init__(self, fn: Any) -> None:
        super().__init__(fn.__globals__)
        self.update(inspect.getclosurevars(fn).nonlocals)

    def __missing__(self, name: str) -> Any:
        if not name[:1].isupper():
            raise KeyError(name)
        return getattr(sym, name)


def resolved_annotations(fn: Any) -> dict[str, Any]:
    """The kernel's parameter annotations with string annotations evaluated
    (hc/simulator.py:664-700 semantics)."""
    raw = inspect.get_annotations(fn, eval_str=False)
    pending = {name: text for name, text in raw.items() if isinstance(text, str)}
    if not pending:
        return dict(raw)
    namespace = _SymbolFallback(fn)
    out = dict(raw)
    for name, text in pending.items():
        try:
            out[name] = eval(text, fn.__globals__, namespace)  # noqa: S307 - annotation text
        except (NameError, TypeError) as exc:
            raise LaunchError(f"failed to resolve annotations for {fn.__name__}") from exc
    return out


class _Binder:
    """Binds observed argument extents to the symbols of their annotations,
    raising the reference's LaunchError texts (hc/simulator.py:780-842)."""

    def __init__(self) -> None:
        self.bindings = Bindings()

    def extent(self, dim: Any, value: int, where: str) -> None:
        """One annotated extent `dim` (symbol, expression or int) observed as `value`."""
        if isinstance(dim, Symbol):
            self.bindings.bind(dim, value, source=where)
        elif isinstance(dim, Expr):
            self.bindings.require(dim, value, source=where)
        elif isinstance(dim, int) and not isinstance(dim, bool) and dim != value:
            raise LaunchError(f"{where} expected {dim}, got {value}")

    def shape(self, dims: tuple[Any, ...], shape: tuple[int, ...], where: str) -> None:
        for index, (dim, value) in enumerate(zip(dims, shape)):
            self.extent(dim, int(value), f"{where}.shape[{index}]")

    def buffer(self, spec: BufferSpec, value: Any, where: str) -> None:
        dtype = buffer_dtype_name(value)
        if dtype is None:
            raise LaunchError(f"{where} must be a numpy.ndarray or torch.Tensor buffer")
        shape = tuple(int(d) for d in value.shape)
        if len(shape) != len(spec.dimensions):
            raise LaunchError(f"{where} rank does not match its Buffer annotation")
        if spec.dtype is not None and dtype != spec.dtype:
            raise LaunchError(f"{where} dtype expected {spec.dtype}, got {dtype}")
        self.shape(spec.dimensions, shape, where)

    def items(self, dims: tuple[Any, ...], value: Any, where: str) -> None:
        if not isinstance(value, tuple):
            raise LaunchError(f"{where} must be a tuple")
        if len(value) != len(dims):
            raise LaunchError(f"{where} length does not match its tuple annotation")
        for index, (dim, item) in enumerate(zip(dims, value)):
            self.extent(dim, int(item), f"{where}[{index}]")


def _resolve_dim(value: Any, env: Env, literal_names: frozenset[str], *, static: bool, name: str) -> int:
    import numpy as np

    if isinstance(value, bool):
        raise LaunchError(f"{name} must be an integer")
    if isinstance(value, (int, np.integer)):
        return int(value)
    if isinstance(value, Expr):
        if static and not {s.name for s in value.free_symbols()} <= literal_names:
            raise LaunchError(f"{name} must be constant or use only literal symbols")
        return int(value.eval(env))
    raise LaunchError(f"{name} must be an integer expression")


def _resolve_shape(spec: Any, env: Env, literal_names: frozenset[str]) -> tuple[int, ...]:
    if spec is None:
        raise LaunchError("kernel metadata is missing required work_shape")
    values = spec if isinstance(spec, tuple) else (spec,)
    return tuple(_resolve_dim(v, env, literal_names, static=False, name="shape") for v in values)


def _validate(work: tuple[int, ...], group: tuple[int, ...], subgroup: int | None, limit: int | None) -> None:
    if len(work) != len(group):
        raise LaunchError("work_shape and group_shape must have the same rank")
    if any(d < 0 for d in work):
        raise LaunchError("work_shape values must be non-negative")
    if any(d <= 0 for d in group):
        raise LaunchError("group_shape values must be positive")
    if subgroup is not None:
        if subgroup <= 0:
            raise LaunchError("subgroup_size must be positive")
        if group and group[0] % subgroup != 0:
            raise LaunchError("group_shape[0] must be divisible by subgroup_size")
    if limit is not None:
        size = 1
        for d in group:
            size *= d
        if size > limit:
            raise LaunchError("group size exceeds the target limit")


def _align_up(value: int, align: int) -> int:
    return -(-value // align) * align


def default_group_shape(work_shape: tuple[int, ...], subgroup_size: int | None) -> tuple[int, ...]:
    """Default group shape when a kernel gives none (hc/simulator.py:67-73)."""
    base = tuple(max(1, d) for d in work_shape)
    if not base or subgroup_size is None:
        return base
    return (_align_up(base[0], subgroup_size), *base[1:])


@dataclass(frozen=True)
class LaunchGeometry:
    env: Env
    literal_names: frozenset[str]
    work_shape: tuple[int, ...]
    group_shape: tuple[int, ...]
    subgroup_size: int | None


def _geometry(metadata: KernelMetadata, env: Env, target: Any) -> LaunchGeometry:
    literal_names = frozenset(s.name for s in metadata.literals if isinstance(s, Symbol))
    work_shape = _resolve_shape(metadata.work_shape, env, literal_names)
    subgroup_size = (
        None
        if metadata.subgroup_size is None
        else _resolve_dim(metadata.subgroup_size, env, literal_names, static=True, name="subgroup_size")
    )
    if metadata.group_shape is None:
        chooser = getattr(target, "choose_group_shape", None)
        group_shape = (
            chooser(work_shape, subgroup_size)
            if chooser is not None
            else default_group_shape(work_shape, subgroup_size)
        )
    else:
        group_shape = _resolve_shape(metadata.group_shape, env, literal_names)
    _validate(work_shape, group_shape, subgroup_size, getattr(target, "max_group_size", None))
    return LaunchGeometry(env, literal_names, work_shape, group_shape, subgroup_size)


def launch_geometry(fn: Any, shapes: dict[str, tuple[int, ...]], target: Any = None) -> LaunchGeometry:
    """Geometry of a launch whose Buffer parameters have the given shapes
    (no argument values: used to plan a launch before buffers exist)."""
    try:
        metadata = kernel_metadata(fn)
        annotations = resolved_annotations(fn)
        binder = _Binder()
        for name, shape in shapes.items():
            spec = annotations.get(name)
            if not isinstance(spec, BufferSpec) or len(spec.dimensions) != len(shape):
                raise LaunchError(f"{name} is not a Buffer of rank {len(shape)}")
            binder.shape(spec.dimensions, shape, name)
        return _geometry(metadata, binder.bindings.freeze(), target)
    except SymbolError as exc:
        raise LaunchError(str(exc)) from exc


def prepare_launch(fn: Any, args: tuple[Any, ...], kwargs: dict[str, Any], target: Any) -> PreparedLaunch:
    try:
        metadata = kernel_metadata(fn)
        bound = _bind_arguments(fn, args, kwargs)
        annotations = resolved_annotations(fn)
        binder = _Binder()
        buffer_params: list[str] = []
        for name, value in bound.arguments.items():
            annotation = annotations.get(name, inspect.Signature.empty)
            if isinstance(annotation, BufferSpec):
                binder.buffer(annotation, value, name)
                buffer_params.append(name)
            elif get_origin(annotation) is tuple:
                binder.items(get_args(annotation), value, name)
        geometry = _geometry(metadata, binder.bindings.freeze(), target)
    except SymbolError as exc:
        raise LaunchError(str(exc)) from exc
    return PreparedLaunch(
        fn=fn,
        bound=bound,
        env=geometry.env,
        literal_names=geometry.literal_names,
        work_shape=geometry.work_shape,
        group_shape=geometry.group_shape,
        subgroup_size=geometry.subgroup_size,
        buffer_params=tuple(buffer_params),
    )
