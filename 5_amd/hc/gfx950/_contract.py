"""Recognition of the tiled contraction that the gfx950 target lowers.

The gfx950 backend does not interpret a kernel: it runs one hand-written
GEMM (libhcg_gfx950.so) in place of the whole launch.  That is only correct
when the kernel *is* that GEMM, so a kernel is accepted only after two checks:

1. **Structure (AST).**  The body must be the canonical tiled contraction of
   examples/amdgpu_gfx11_wmma_matmul.py:306-326, statement for statement::

       row0, col0 = <tile origin of group.group_id>
       acc = <init helper>(group)
       for k0 in range(0, a.shape[1], TK):
           a_tile = group.load(a[row0 : row0 + TM, k0 : k0 + TK], shape=(TM, TK))
           b_tile = group.load(b[k0 : k0 + TK, col0 : col0 + TN], shape=(TK, TN))
           acc = <accumulate helper>(group, a_tile, b_tile, acc)
       <store helper>(group, c, row0, col0, acc)

   with TM, TN, TK integer constants, the loop step equal to the loaded K
   extent, the helpers ``@kernel.func`` functions, and ``a``, ``b``, ``c``
   the kernel's ``Buffer[M, K, T]``, ``Buffer[K, N, T]`` and
   ``Buffer[M, N, float32]`` parameters (T float16 or bfloat16).

2. **Semantics (a recorded run).**  Every workgroup of a small ragged launch
   (M, N, K one and a half tiles plus one, so every tail is masked) runs on
   the CPU through the kernel's own helpers and intrinsic fallback bodies,
   with the reference simulator's rules for what they touch
   (hc/simulator.py:302-358 load/store/vzeros/vload, :560-645 workitems run
   in dimension-0-fastest order, :1090-1288 collective returns lifted over
   the group shape, :1338-1357 loads copy the in-bounds overlap and mask the
   rest, :1441-1458 stores write active elements of the overlap;
   hc/_sim_types.py:287-357 indexing, ``vec``, ``with_inactive``, and reading
   an inactive element is an error).  Each call of an intrinsic is checked
   as the simulator checks it (hc/simulator.py:972-1001: declared scope, a
   fallback body, the verify hook) and must also carry a lowering registered
   for ``amdgpu-gfx950`` (``mfma_gfx950``, ``mfma16_gfx950``) or
   ``amdgpu-gfx11`` (the reference's ``wmma_gfx11``).  That lowering callback
   is called, once per call site, with a recording ``ctx`` (``_lowering``):
   the op it creates must be a matrix-core instruction this library executes
   (``rocdl.mfma.f32.32x32x16`` / ``16x16x32``, or the reference's
   ``amdgpu.wmma``), with matching ``m``/``n``/``k``/``arch``/``wave_size``,
   a float32 vector result and the accumulator as its last operand, and its
   m x n x k must be the kernel's tile and K step (one op per lane and K
   step computes the tile) for waves of the workgroup's size.  The GPU
   kernel replaces the whole loop of them.  The inputs are integers, so every
   summation order is exact and C must equal A @ B exactly; an element left
   unwritten (C starts as NaN) or any other value rejects the kernel.  Two
   runs are made: one with small values, and one (one workgroup's tile, K
   one and a half steps plus one) whose partial sums reach ~10^6, which
   only float32 accumulation computes exactly (the reference folds in
   np.float32, examples/amdgpu_gfx11_wmma_matmul.py:183-190); the
   accumulator the init and accumulate helpers return must be float32.

A kernel that fails either check raises ``LaunchError`` naming it and the
reason.  Results are cached per kernel function.  The check runs the
kernel's Python code on one small launch; a helper whose behaviour depends
on the problem size beyond that launch is not covered.
"""

from __future__ import annotations

import ast
import inspect
import sys
import textwrap
import threading
from collections.abc import Callable, Iterator
from dataclasses import dataclass
from typing import Any

import numpy as np

from .._errors import LaunchError
from .._launch import launch_geometry, resolved_annotations
from ._lowering import TARGET_ARCH, TARGET_ORDER, Location, LoweringError, check_matrix_op, lowering_target, record_lowering
from ..core import BufferSpec, WorkGroup, WorkItem
from ..symbols import Expr, Symbol

TARGET_NAME = "amdgpu-gfx950"
_ELEMENT_TYPES = ("float16", "bfloat16")


@dataclass(frozen=True)
class Contraction:
    """A kernel recognised as C = A @ B."""

    a: str  # parameter names of the A, B and C buffers
    b: str
    c: str
    dtype: str  # "float16" or "bfloat16"
    tile: tuple[int, int, int]  # (TM, TN, TK) of one workgroup's tile and K step
    intrinsics: tuple[str, ...]  # intrinsics the recorded run called
    ops: tuple[str, ...] = ()  # the ops their lowerings create (recorded through a ctx)


class _Reject(Exception):
    """Internal: the kernel is not the contraction (message says why)."""


def gemm_signature(fn: Any) -> tuple[str, str, str, str] | None:
    """(a, b, c, dtype) if ``fn``'s buffers form ``(Buffer[M, K, T],
    Buffer[K, N, T], Buffer[M, N, float32])`` with M, N, K three distinct
    symbols and T float16 or bfloat16, else None."""
    try:
        annotations = resolved_annotations(fn)
    except LaunchError:
        return None
    specs = [(name, spec) for name, spec in annotations.items() if isinstance(spec, BufferSpec)]
    if len(specs) != 3:
        return None
    (na, a), (nb, b), (nc, c) = specs
    if not all(len(s.dimensions) == 2 for s in (a, b, c)):
        return None
    if not all(isinstance(d, Symbol) for s in (a, b, c) for d in s.dimensions):
        return None
    m, k = a.dimensions
    k2, n = b.dimensions
    m2, n2 = c.dimensions
    if not (k == k2 and m == m2 and n == n2) or len({m, n, k}) != 3:
        return None
    if a.dtype != b.dtype or a.dtype not in _ELEMENT_TYPES or c.dtype != "float32":
        return None
    return na, nb, nc, a.dtype


# --------------------------------------------------------------------------
# 1. Structure
# --------------------------------------------------------------------------


def _const(node: ast.AST, env: dict[str, Any]) -> int:
    """Integer value of a constant expression (literals, module names bound
    to ints, + - * //); anything else is not a tile constant."""
    if isinstance(node, ast.Constant) and isinstance(node.value, int) and not isinstance(node.value, bool):
        return node.value
    if isinstance(node, ast.Name):
        value = env.get(node.id)
        if isinstance(value, (int, np.integer)) and not isinstance(value, bool):
            return int(value)
        raise _Reject(f"{node.id!r} is not an integer constant")
    if isinstance(node, ast.BinOp) and isinstance(node.op, (ast.Add, ast.Sub, ast.Mult, ast.FloorDiv)):
        lhs, rhs = _const(node.left, env), _const(node.right, env)
        if isinstance(node.op, ast.Add):
            return lhs + rhs
        if isinstance(node.op, ast.Sub):
            return lhs - rhs
        if isinstance(node.op, ast.Mult):
            return lhs * rhs
        if rhs == 0:
            raise _Reject("division by zero in a tile constant")
        return lhs // rhs
    raise _Reject(f"{ast.unparse(node)!r} is not an integer constant")


def _name(node: ast.AST) -> str | None:
    return node.id if isinstance(node, ast.Name) else None


def _helper(node: ast.AST, env: dict[str, Any], what: str) -> str:
    name = _name(node)
    fn = env.get(name) if name else None
    if fn is None or not hasattr(fn, "__hc_func__"):
        raise _Reject(f"the {what} must call a @kernel.func helper by name")
    return name


def _plain_call(node: ast.AST) -> ast.Call:
    if not isinstance(node, ast.Call) or node.keywords or any(isinstance(a, ast.Starred) for a in node.args):
        raise _Reject(f"expected a plain call, got {ast.unparse(node)!r}")
    return node


def _args_are(call: ast.Call, names: tuple[str, ...]) -> bool:
    return tuple(_name(arg) for arg in call.args) == names


def _tile_slice(node: ast.AST, origin: str, env: dict[str, Any]) -> int:
    """Extent E of ``origin : origin + E`` (no step)."""
    if not isinstance(node, ast.Slice) or node.step is not None or _name(node.lower) != origin:
        raise _Reject(f"expected the slice {origin} : {origin} + <tile>")
    upper = node.upper
    if not (isinstance(upper, ast.BinOp) and isinstance(upper.op, ast.Add) and _name(upper.left) == origin):
        raise _Reject(f"expected the slice {origin} : {origin} + <tile>")
    return _const(upper.right, env)


def _tile_load(stmt: ast.stmt, group: str, env: dict[str, Any]) -> tuple[str, str, tuple[ast.AST, ast.AST], tuple[int, int]]:
    """(tile name, buffer name, the two slices, shape=) of
    ``t = group.load(buf[s0, s1], shape=(e0, e1))``."""
    if not (isinstance(stmt, ast.Assign) and len(stmt.targets) == 1 and _name(stmt.targets[0])):
        raise _Reject("the K loop must first load two tiles with group.load")
    call = stmt.value
    if not (
        isinstance(call, ast.Call)
        and isinstance(call.func, ast.Attribute)
        and call.func.attr == "load"
        and _name(call.func.value) == group
        and len(call.args) == 1
        and len(call.keywords) == 1
        and call.keywords[0].arg == "shape"
    ):
        raise _Reject("tiles must be loaded as group.load(buffer[...], shape=(rows, cols))")
    src = call.args[0]
    if not (isinstance(src, ast.Subscript) and _name(src.value) and isinstance(src.slice, ast.Tuple) and len(src.slice.elts) == 2):
        raise _Reject("a tile load must slice a buffer in two dimensions")
    shape = call.keywords[0].value
    if not (isinstance(shape, ast.Tuple) and len(shape.elts) == 2):
        raise _Reject("shape= of a tile load must be a pair")
    extents = (_const(shape.elts[0], env), _const(shape.elts[1], env))
    return _name(stmt.targets[0]), _name(src.value), (src.slice.elts[0], src.slice.elts[1]), extents


def _function_node(fn: Any) -> ast.FunctionDef:
    try:
        source = textwrap.dedent(inspect.getsource(fn))
    except (OSError, TypeError) as exc:
        raise _Reject("its source is not available") from exc
    tree = ast.parse(source)
    node = tree.body[0] if tree.body else None
    if not isinstance(node, ast.FunctionDef):
        raise _Reject("its definition was not found in its source")
    return node


def _check_structure(fn: Any, a: str, b: str, c: str) -> tuple[tuple[int, int, int], tuple[Any, Any]]:
    """Checks the body's statements; returns (TM, TN, TK) and the init and
    accumulate helpers."""
    node = _function_node(fn)
    params = [arg.arg for arg in node.args.args]
    if node.args.vararg or node.args.kwarg or node.args.kwonlyargs or node.args.posonlyargs:
        raise _Reject("it takes parameters besides the group and three buffers")
    if len(params) != 4 or set(params[1:]) != {a, b, c}:
        raise _Reject("its parameters must be the group and the three buffers")
    group = params[0]
    env = dict(fn.__globals__)
    closure = inspect.getclosurevars(fn)
    env.update(closure.nonlocals)

    body = list(node.body)
    if body and isinstance(body[0], ast.Expr) and isinstance(body[0].value, ast.Constant) and isinstance(body[0].value.value, str):
        body = body[1:]
    if body and (isinstance(body[-1], ast.Pass) or (isinstance(body[-1], ast.Return) and (body[-1].value is None or (isinstance(body[-1].value, ast.Constant) and body[-1].value.value is None)))):
        body = body[:-1]
    if len(body) != 4:
        raise _Reject("the body must be: tile origin, accumulator init, K loop, store")
    origin, init, loop, store = body

    # row0, col0 = <expression of the group id>
    if not (
        isinstance(origin, ast.Assign)
        and len(origin.targets) == 1
        and isinstance(origin.targets[0], ast.Tuple)
        and len(origin.targets[0].elts) == 2
        and all(_name(e) for e in origin.targets[0].elts)
    ):
        raise _Reject("the first statement must assign the tile origin pair (row0, col0)")
    row0, col0 = (_name(e) for e in origin.targets[0].elts)
    used = {n.id for n in ast.walk(origin.value) if isinstance(n, ast.Name)}
    if used & {a, b, c}:
        raise _Reject("the tile origin may not depend on the buffers")

    # acc = init(group)
    if not (isinstance(init, ast.Assign) and len(init.targets) == 1 and _name(init.targets[0])):
        raise _Reject("the second statement must initialise the accumulator")
    acc = _name(init.targets[0])
    init_call = _plain_call(init.value)
    init_helper = _helper(init_call.func, env, "accumulator init")
    if not _args_are(init_call, (group,)):
        raise _Reject("the accumulator init must take only the group")

    # for k0 in range(0, a.shape[1], TK): two loads, one accumulate
    if not (isinstance(loop, ast.For) and _name(loop.target) and not loop.orelse):
        raise _Reject("the third statement must be the K loop")
    k = _name(loop.target)
    it = loop.iter
    if not (isinstance(it, ast.Call) and _name(it.func) == "range" and len(it.args) == 3 and not it.keywords):
        raise _Reject("the K loop must be range(0, a.shape[1], <tile K>)")
    start, stop, step_node = it.args
    if not (isinstance(start, ast.Constant) and start.value == 0):
        raise _Reject("the K loop must start at 0")
    if not (
        isinstance(stop, ast.Subscript)
        and isinstance(stop.value, ast.Attribute)
        and stop.value.attr == "shape"
        and _name(stop.value.value) == a
        and isinstance(stop.slice, ast.Constant)
        and stop.slice.value == 1
    ):
        raise _Reject(f"the K loop must run to {a}.shape[1]")
    step = _const(step_node, env)
    if step <= 0:
        raise _Reject("the K step must be positive")
    if len(loop.body) != 3:
        raise _Reject("the K loop body must be two tile loads and one accumulate")
    loads = [_tile_load(s, group, env) for s in loop.body[:2]]
    by_buffer = {load[1]: load for load in loads}
    if set(by_buffer) != {a, b}:
        raise _Reject(f"the K loop must load one tile of {a} and one of {b}")
    ta, _, (sa0, sa1), (tm, tk_a) = by_buffer[a]
    tb, _, (sb0, sb1), (tk_b, tn) = by_buffer[b]
    if _tile_slice(sa0, row0, env) != tm or _tile_slice(sa1, k, env) != tk_a:
        raise _Reject(f"the {a} tile must be {a}[{row0} : {row0} + TM, {k} : {k} + TK] with shape=(TM, TK)")
    if _tile_slice(sb0, k, env) != tk_b or _tile_slice(sb1, col0, env) != tn:
        raise _Reject(f"the {b} tile must be {b}[{k} : {k} + TK, {col0} : {col0} + TN] with shape=(TK, TN)")
    if not (tk_a == tk_b == step):
        raise _Reject(f"the K step ({step}) must equal the tiles' K extent ({tk_a}, {tk_b})")
    if min(tm, tn, step) <= 0:
        raise _Reject("tile extents must be positive")
    accumulate = loop.body[2]
    if not (isinstance(accumulate, ast.Assign) and len(accumulate.targets) == 1 and _name(accumulate.targets[0]) == acc):
        raise _Reject(f"the K loop must end with {acc} = <accumulate>(group, a_tile, b_tile, {acc})")
    acc_call = _plain_call(accumulate.value)
    acc_helper = _helper(acc_call.func, env, "accumulate step")
    if not _args_are(acc_call, (group, ta, tb, acc)):
        raise _Reject(f"the accumulate step must take ({group}, {ta}, {tb}, {acc})")
    if len({row0, col0, acc, k, ta, tb, group, a, b, c}) != 10:
        raise _Reject("the origin, accumulator, loop and tile names must be distinct")

    # store(group, c, row0, col0, acc)
    if not isinstance(store, ast.Expr):
        raise _Reject("the last statement must store the accumulator")
    store_call = _plain_call(store.value)
    _helper(store_call.func, env, "store")
    if not _args_are(store_call, (group, c, row0, col0, acc)):
        raise _Reject(f"the store must take ({group}, {c}, {row0}, {col0}, {acc})")
    return (tm, tn, step), (env[init_helper], env[acc_helper])


# --------------------------------------------------------------------------
# 2. Recorded run
# --------------------------------------------------------------------------


class _Masked:
    """Payload + activity mask (the simulator's SimTensor / SimVector)."""

    __slots__ = ("_data", "_mask", "kind")

    def __init__(self, data: np.ndarray, mask: np.ndarray, kind: str) -> None:
        self._data = data
        self._mask = mask
        self.kind = kind

    @property
    def shape(self) -> tuple[int, ...]:
        return tuple(int(d) for d in self._data.shape)

    @property
    def dtype(self) -> np.dtype:
        return self._data.dtype

    @property
    def ndim(self) -> int:
        return self._data.ndim

    @property
    def mask(self) -> _Masked:
        return _Masked(self._mask.copy(), np.ones(self._mask.shape, dtype=bool), self.kind)

    def __getitem__(self, index: Any) -> Any:
        data = self._data[index]
        mask = self._mask[index]
        if isinstance(mask, np.bool_):
            if not mask:
                raise _Reject("it reads an inactive (masked-off) element")
            return data
        return _Masked(data, mask, self.kind)

    def with_inactive(self, *, value: Any) -> _Masked:
        fill = np.asarray(value, dtype=self._data.dtype)
        return _Masked(np.where(self._mask, self._data, fill), np.ones(self._mask.shape, dtype=bool), self.kind)

    def vec(self, shape: Any = None) -> _Masked:
        resolved = self.shape if shape is None else tuple(int(d) for d in shape)
        return _Masked(self._data.reshape(resolved), self._mask.reshape(resolved), "vector")

    def __array__(self, *args: Any, **kwargs: Any) -> np.ndarray:
        raise TypeError("tile values do not convert to numpy arrays implicitly")

    def __bool__(self) -> bool:
        raise TypeError("tile values do not define truthiness")


class _ValueSig:
    """What a verify hook sees of one argument (hc/simulator.py:85-113)."""

    def __init__(self, value: Any) -> None:
        self.value = value

    @property
    def type(self) -> Any:
        return self.value.dtype if hasattr(self.value, "dtype") else type(self.value)

    @property
    def shape(self) -> tuple[int, ...] | None:
        return tuple(int(d) for d in self.value.shape) if hasattr(self.value, "shape") else None

    @property
    def mask(self) -> Any:
        return getattr(self.value, "mask", None)

    @property
    def layout(self) -> Any:
        return None

    def is_tensor(self) -> bool:
        return isinstance(self.value, _Masked) and self.value.kind == "tensor"

    def is_vector(self) -> bool:
        return isinstance(self.value, _Masked) and self.value.kind == "vector"

    def is_buffer(self) -> bool:
        return isinstance(self.value, np.ndarray)


class _CallSig:
    """The verify hook's call signature (hc/simulator.py:116-130)."""

    def __init__(self, scope: Any, args: tuple[Any, ...], kwargs: dict[str, Any]) -> None:
        self.scope = scope
        self._args = args
        self._kwargs = kwargs

    def arg(self, index: int) -> Any:
        value = self._args[index]
        return _ValueSig(value) if isinstance(value, (_Masked, np.ndarray)) else value

    def kwarg(self, name: str) -> Any:
        return self._kwargs.get(name)


class _WorkItem(WorkItem):
    def __init__(self, local_id: tuple[int, ...], global_id: tuple[int, ...]) -> None:
        self._local = local_id
        self._global = global_id

    def local_id(self) -> tuple[int, ...]:
        return self._local

    def global_id(self) -> tuple[int, ...]:
        return self._global


def _indices(shape: tuple[int, ...]) -> Iterator[tuple[int, ...]]:
    """Dimension 0 fastest (hc/simulator.py:1298-1301)."""
    for rev in np.ndindex(tuple(reversed(shape))):
        yield tuple(reversed(rev))


def _lift(results: list[tuple[tuple[int, ...], Any]], shape: tuple[int, ...]) -> Any:
    """Collective return of a workitem region over the group shape
    (hc/simulator.py:1090-1288): None, scalars, vectors and flat tuples."""
    first = results[0][1]
    if first is None:
        if any(v is not None for _, v in results):
            raise _Reject("a workitem region returns None from some workitems only")
        return None
    if isinstance(first, tuple):
        return tuple(_lift([(i, v[p]) for i, v in results], shape) for p in range(len(first)))
    if isinstance(first, _Masked):
        if first.kind != "vector":
            raise _Reject("a workitem region returns a tensor")
        data = np.zeros(first.shape + shape, dtype=first.dtype)
        mask = np.zeros(first.shape + shape, dtype=bool)
        lead = (slice(None),) * len(first.shape)
        for index, value in results:
            if not isinstance(value, _Masked) or value.shape != first.shape or value.dtype != first.dtype:
                raise _Reject("workitem returns differ in structure")
            data[lead + index] = value._data
            mask[lead + index] = value._mask
        return _Masked(data, mask, "vector")
    if np.isscalar(first):
        data = np.zeros(shape, dtype=np.asarray(first).dtype)
        for index, value in results:
            data[index] = value
        return _Masked(data, np.ones(shape, dtype=bool), "vector")
    raise _Reject(f"a workitem region returns {type(first).__name__}")


def _copy_overlap(source: Any, shape: tuple[int, ...], kind: str) -> _Masked:
    if isinstance(source, _Masked):
        src, src_mask = source._data, source._mask
    elif isinstance(source, np.ndarray):
        src, src_mask = source, np.ones(source.shape, dtype=bool)
    else:
        raise _Reject("a load source must be a buffer view or a tile value")
    if src.ndim != len(shape):
        raise _Reject("load rank does not match shape=")
    data = np.zeros(shape, dtype=src.dtype)
    mask = np.zeros(shape, dtype=bool)
    overlap = tuple(slice(0, min(shape[i], src.shape[i])) for i in range(len(shape)))
    data[overlap] = src[overlap]
    mask[overlap] = src_mask[overlap]
    return _Masked(data, mask, kind)


class _Group:
    """The workgroup handle of the recorded run (hc/simulator.py:235-511)."""

    def __init__(self, run: _Run, group_id: tuple[int, ...], shape: tuple[int, ...], work_shape: tuple[int, ...]) -> None:
        self._run = run
        self.group_id = group_id
        self.shape = shape
        self.work_shape = work_shape
        self.work_offset = tuple(g * s for g, s in zip(group_id, shape))

    @property
    def size(self) -> int:
        return int(np.prod(self.shape))

    def _dims(self, shape: Any) -> tuple[int, ...]:
        if shape is None:
            raise _Reject("shape= is required")
        out = []
        for d in shape:
            if isinstance(d, Expr):
                d = d.eval(self._run.env)
            if not isinstance(d, (int, np.integer)) or isinstance(d, bool):
                raise _Reject("shape= entries must be integers")
            out.append(int(d))
        return tuple(out)

    def _load(self, source: Any, shape: Any, mask: Any, kind: str) -> _Masked:
        if (shape is None) == (mask is None):
            raise _Reject("a load needs exactly one of shape= or mask=")
        if mask is not None:
            if not isinstance(mask, _Masked) or mask.dtype != np.dtype(bool):
                raise _Reject("mask= must be a bool tile value")
            loaded = _copy_overlap(source, mask.shape, kind)
            return _Masked(loaded._data, loaded._mask & mask._mask & mask._data, kind)
        return _copy_overlap(source, self._dims(shape), kind)

    def load(self, source: Any, *, shape: Any = None, mask: Any = None, layout: Any = None) -> _Masked:
        self._run.require_group_scope("group.load()")
        return self._load(source, shape, mask, "tensor")

    def vload(self, source: Any, *, shape: Any = None, mask: Any = None, layout: Any = None) -> _Masked:
        return self._load(source, shape, mask, "vector")

    def store(self, target: Any, value: Any) -> None:
        if isinstance(value, _Masked) and value.kind == "tensor":
            self._run.require_group_scope("group.store() with a tensor source")
        if not isinstance(target, np.ndarray):
            raise _Reject("stores must target a buffer view")
        if isinstance(value, _Masked):
            if value.ndim != target.ndim:
                raise _Reject("store source and target ranks differ")
            overlap = tuple(slice(0, min(target.shape[i], value.shape[i])) for i in range(target.ndim))
            region = target[overlap]
            src_mask = value._mask[overlap]
            region[src_mask] = value._data[overlap][src_mask]
        else:
            target[...] = value

    def _alloc(self, shape: Any, dtype: Any, fill: Any, active: bool, kind: str) -> _Masked:
        dims = self._dims(shape)
        return _Masked(np.full(dims, fill, dtype=np.dtype(dtype)), np.full(dims, active, dtype=bool), kind)

    def vzeros(self, *, shape: Any, dtype: Any, layout: Any = None) -> _Masked:
        return self._alloc(shape, dtype, 0, True, "vector")

    def vones(self, *, shape: Any, dtype: Any, layout: Any = None) -> _Masked:
        return self._alloc(shape, dtype, 1, True, "vector")

    def vfull(self, *, shape: Any, dtype: Any, fill_value: Any, layout: Any = None) -> _Masked:
        return self._alloc(shape, dtype, fill_value, True, "vector")

    def zeros(self, *, shape: Any, dtype: Any, layout: Any = None) -> _Masked:
        self._run.require_group_scope("group.zeros()")
        return self._alloc(shape, dtype, 0, True, "tensor")

    def full(self, *, shape: Any, dtype: Any, fill_value: Any, layout: Any = None) -> _Masked:
        self._run.require_group_scope("group.full()")
        return self._alloc(shape, dtype, fill_value, True, "tensor")

    def empty(self, *, shape: Any, dtype: Any, layout: Any = None) -> _Masked:
        self._run.require_group_scope("group.empty()")
        return self._alloc(shape, dtype, 0, False, "tensor")

    def barrier(self) -> None:
        raise _Reject("it uses group.barrier(), which the contraction check does not model")

    def subgroups(self, fn: Callable[..., Any]) -> Callable[..., Any]:
        raise _Reject("it uses @group.subgroups, which the contraction check does not model")

    def workitems(self, fn: Callable[..., Any]) -> Callable[..., Any]:
        def region(*args: Any, **kwargs: Any) -> Any:
            if args or kwargs:
                raise _Reject("collective region runners take no call-time arguments")
            self._run.require_group_scope("@group.workitems")
            results = []
            for local in _indices(self.shape):
                wi = _WorkItem(local, tuple(o + l for o, l in zip(self.work_offset, local)))
                self._run.scope = WorkItem
                try:
                    results.append((local, fn(wi)))
                finally:
                    self._run.scope = WorkGroup
            return _lift(results, self.shape)

        return region


_ACTIVE = threading.local()


class _Run:
    """State of one recorded run: scope, intrinsic calls, the first error."""

    def __init__(self, env: Any, target: Any) -> None:
        self.env = env
        self.target = target
        self.scope: Any = WorkGroup
        self.intrinsic_calls = 0
        self.intrinsics: set[str] = set()
        self.error: str | None = None
        self.codes: dict[Any, Any] = {}  # code object -> hc helper / intrinsic, or None
        self.acc_codes: dict[Any, str] = {}  # code object of the init / accumulate helper -> its name
        # intrinsic call site -> (lowered op, its (m, n, k), its wave size)
        self.lowered: dict[Any, tuple[str, tuple[int, int, int], int]] = {}

    def require_group_scope(self, what: str) -> None:
        if self.scope is not WorkGroup:
            raise _Reject(f"{what} is used outside WorkGroup scope")

    def fail(self, message: str) -> None:
        if self.error is None:
            self.error = message

    def check_scope(self, kind: str, fn: Any, declared: Any) -> None:
        if declared is None:
            return
        if declared is not WorkGroup and declared is not WorkItem:
            self.fail(f"{kind} {fn.__name__!r} declares scope {declared!r}, which the check does not model")
        elif declared is not self.scope:
            self.fail(f"{kind} {fn.__name__!r} runs in {self.scope.__name__ if self.scope is WorkItem else 'WorkGroup'} "
                      f"scope but declares {declared.__name__ if declared is WorkItem else 'WorkGroup'}")

    def on_accumulator(self, name: str, value: Any) -> None:
        """The kernel's accumulator must be float32, as the reference's is
        (examples/amdgpu_gfx11_wmma_matmul.py:183-190 folds in np.float32):
        the GPU kernels accumulate in float32 whatever the helpers do."""
        if not isinstance(value, _Masked):
            self.fail(f"helper {name!r} returns {type(value).__name__}, not a float32 accumulator")
        elif value.dtype != np.dtype(np.float32):
            self.fail(f"helper {name!r} returns a {value.dtype} accumulator, not float32")

    def on_intrinsic(self, fn: Any, frame: Any) -> None:
        self.check_scope("intrinsic", fn, fn.__hc_intrinsic__.scope)
        if not getattr(fn, "__hc_has_fallback__", False):
            self.fail(f"intrinsic {fn.__name__!r} has no fallback body")
            return
        lowerings = getattr(fn, "__hc_lowerings__", {}) or {}
        if not any(str(t).startswith("amdgpu-") for t in lowerings):
            self.fail(f"intrinsic {fn.__name__!r} has no lowering registered for an amdgpu target")
            return
        target = lowering_target(fn)
        if target is None:
            self.fail(f"intrinsic {fn.__name__!r} has lowerings for {', '.join(sorted(map(str, lowerings)))}, "
                      f"none of which this library executes ({', '.join(TARGET_ORDER)})")
            return
        self.intrinsic_calls += 1
        self.intrinsics.add(fn.__name__)
        args: list[Any] = []
        kwargs: dict[str, Any] = {}
        local = frame.f_locals
        for param in inspect.signature(fn).parameters.values():
            if param.kind in (param.POSITIONAL_ONLY, param.POSITIONAL_OR_KEYWORD):
                args.append(local[param.name])
            elif param.kind is param.VAR_POSITIONAL:
                args.extend(local.get(param.name, ()))
            elif param.kind is param.KEYWORD_ONLY:
                kwargs[param.name] = local[param.name]
            else:
                kwargs.update(local.get(param.name, {}))
        verify = getattr(fn, "__hc_verify__", None)
        if verify is not None:
            try:
                result = verify(_CallSig(self.scope, tuple(args), kwargs), self.target)
            except Exception as exc:  # noqa: BLE001 - the hook's failure is the verdict
                self.fail(f"intrinsic {fn.__name__!r} verify hook failed: {exc}")
                return
            if result is False:
                self.fail(f"intrinsic {fn.__name__!r} verify hook returned False")
                return
        # The lowering replaces this call on its target: call it as the
        # compiler would and check the op it creates (once per call site).
        caller = frame.f_back
        site = (fn, caller.f_code, caller.f_lineno) if caller is not None else (fn, None, 0)
        if site in self.lowered:
            return
        loc = Location(caller.f_code.co_filename, caller.f_lineno) if caller is not None else None
        try:
            op = record_lowering(fn, target, tuple(args), kwargs, loc)
            shape = check_matrix_op(op, target, fn, tuple(args))
        except LoweringError as exc:
            self.fail(str(exc))
            return
        self.lowered[site] = (op.name, shape, TARGET_ARCH[target][1])


def _profile(frame: Any, event: str, arg: Any) -> None:
    if event == "return":
        run = getattr(_ACTIVE, "run", None)
        if run is not None:
            name = run.acc_codes.get(frame.f_code)
            if name is not None:
                run.on_accumulator(name, arg)
        return
    if event != "call":
        return
    run = getattr(_ACTIVE, "run", None)
    if run is None:
        return
    code = frame.f_code
    fn = run.codes.get(code, _UNSEEN)
    if fn is _UNSEEN:
        fn = frame.f_globals.get(code.co_name)
        if fn is None or getattr(fn, "__code__", None) is not code or not (
            hasattr(fn, "__hc_intrinsic__") or hasattr(fn, "__hc_func__")
        ):
            fn = None
        run.codes[code] = fn
    if fn is None:
        return
    if hasattr(fn, "__hc_intrinsic__"):
        run.on_intrinsic(fn, frame)
    else:
        run.check_scope("helper", fn, fn.__hc_func__.scope)


_UNSEEN = object()


# The recorded runs' input ranges.  Every value is an integer the element
# type holds exactly (float16 up to 2048, bfloat16 up to 256) and every
# partial sum stays below 2^24, so float32 accumulation in any order gives
# A @ B exactly.  The first probe's sums stay small (a kernel that is not the
# contraction fails it whatever its arithmetic); the second's reach ~10^6, so
# accumulating in float16 or bfloat16, or clamping, gives other values.
_PROBES = ("small", "wide")


def _probe_inputs(tm: int, tn: int, tk: int, dtype: str, probe: str) -> tuple[np.ndarray, np.ndarray]:
    # The small probe masks every tail (each extent one and a half tiles plus
    # one); the wide one tests the accumulation only: one workgroup's tile,
    # over a K of one and a half K steps plus one.
    m, n, k = (tm + tm // 2 + 1, tn + tn // 2 + 1, tk + tk // 2 + 1) if probe == "small" else (tm, tn, tk + tk // 2 + 1)
    rng = np.random.default_rng(0x5EED if probe == "small" else 0x5EED + 1)
    # bfloat16 kernels see their values as float32 payloads.
    payload = np.float16 if dtype == "float16" else np.float32
    if probe == "small":
        lo = 3
    else:
        lo = 200 if dtype == "float16" else 128
        lo = min(lo, int(np.sqrt((1 << 24) / (2 * k))))
    a = rng.integers(-lo, lo + 1, size=(m, k)).astype(payload)
    b = rng.integers(-lo, lo + 1, size=(k, n)).astype(payload)
    return a, b


def _record(fn: Any, names: tuple[str, str, str], tile: tuple[int, int, int], dtype: str, target: Any,
            helpers: tuple[Any, Any], probe: str) -> tuple[tuple[str, ...], tuple[str, ...]]:
    a_name, b_name, c_name = names
    a, b = _probe_inputs(*tile, dtype, probe)
    m, k = a.shape
    n = b.shape[1]
    c = np.full((m, n), np.nan, dtype=np.float32)
    geometry = launch_geometry(fn, {a_name: a.shape, b_name: b.shape, c_name: c.shape}, target)
    counts = tuple(-(-w // g) for w, g in zip(geometry.work_shape, geometry.group_shape))
    if any(d == 0 for d in counts):
        raise _Reject("its launch geometry is empty for a non-empty problem")
    run = _Run(geometry.env, target)
    for helper in helpers:
        run.acc_codes[helper.__code__] = helper.__name__
    params = list(inspect.signature(fn).parameters)[1:]
    buffers = {a_name: a, b_name: b, c_name: c}
    previous = sys.getprofile()
    _ACTIVE.run = run
    sys.setprofile(_profile)
    try:
        for group_id in _indices(counts):
            fn(_Group(run, group_id, geometry.group_shape, geometry.work_shape), *(buffers[p] for p in params))
            if run.error is not None:
                break
    except _Reject:
        raise
    except Exception as exc:  # noqa: BLE001 - any failure of the body rejects it
        raise _Reject(f"running it on a {m}x{n}x{k} probe raised {type(exc).__name__}: {exc}") from exc
    finally:
        sys.setprofile(previous)
        _ACTIVE.run = None
    if run.error is not None:
        raise _Reject(run.error)
    if run.intrinsic_calls == 0:
        raise _Reject("its accumulate step calls no intrinsic")
    lanes = int(np.prod(geometry.group_shape))
    for op_name, shape, wave in run.lowered.values():
        # One lowered op per lane and K step computes the whole workgroup
        # tile, as the GPU kernels' matrix-core steps do.
        if shape != tile:
            raise _Reject(f"its intrinsic lowers to {op_name} (m x n x k = {shape[0]} x {shape[1]} x {shape[2]}), "
                          f"which does not compute its {tile[0]} x {tile[1]} tile over a K step of {tile[2]}")
        if wave != lanes:
            raise _Reject(f"its intrinsic lowers to {op_name} for {wave}-lane waves, but a workgroup has {lanes} "
                          "workitems")
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    missing = int(np.isnan(c).sum())
    if missing:
        raise _Reject(f"a {m}x{n}x{k} probe leaves {missing} elements of {c_name} unwritten")
    wrong = int((c != want).sum())
    if wrong:
        what = "" if probe == "small" else " with partial sums that need float32 accumulation"
        raise _Reject(f"a {m}x{n}x{k} probe{what} computes {wrong} elements of {c_name} that differ from A @ B")
    return tuple(sorted(run.intrinsics)), tuple(sorted({name for name, _, _ in run.lowered.values()}))


_CACHE: dict[Any, Contraction | str] = {}
_CACHE_LOCK = threading.Lock()


def recognise(fn: Any, target: Any = None) -> Contraction:
    """The kernel's contraction, or ``LaunchError`` naming why it is not one."""
    with _CACHE_LOCK:
        hit = _CACHE.get(fn)
    if hit is None:
        try:
            hit = _recognise(fn, target)
        except _Reject as exc:
            hit = str(exc)
        with _CACHE_LOCK:
            _CACHE[fn] = hit
    if isinstance(hit, str):
        raise LaunchError(f"no {TARGET_NAME} lowering for kernel {getattr(fn, '__name__', fn)!r}: {hit}")
    return hit


def _recognise(fn: Any, target: Any) -> Contraction:
    if not hasattr(fn, "__hc_kernel__"):
        raise _Reject("it is not decorated with @kernel")
    sig = gemm_signature(fn)
    if sig is None:
        raise _Reject("its buffers are not (Buffer[M, K, T], Buffer[K, N, T], Buffer[M, N, float32]) with T "
                      "float16 or bfloat16")
    a, b, c, dtype = sig
    tile, helpers = _check_structure(fn, a, b, c)
    intrinsics: tuple[str, ...] = ()
    ops: tuple[str, ...] = ()
    for probe in _PROBES:
        intrinsics, ops = _record(fn, (a, b, c), tile, dtype, target, helpers, probe)
    return Contraction(a=a, b=b, c=c, dtype=dtype, tile=tile, intrinsics=intrinsics, ops=ops)


def forget(fn: Any) -> None:
    """Drop a cached verdict (after a kernel's helpers changed)."""
    with _CACHE_LOCK:
        _CACHE.pop(fn, None)
