"""Integer symbols for launch geometry: ``sym.M``, ``ceil_div``, ``Bindings``.

The reference backs ``hc.symbols`` with the third-party ``ixsimpl`` symbolic
simplifier (hc/symbols.py, hc/_symbols_backend.py:76-82).  The GEMM launch
only needs the integer subset: binding buffer extents to symbols with
conflict detection (``Bindings.bind``, hc/symbols.py:408-418), checking
derived extents (``Bindings.require``, :430-446), and evaluating the
``work_shape`` expression ``ceil_div(M, 16) * 32`` (``ceil_div``, :499-501;
``Expr.eval``, :226).  This module is a small closed-form integer expression
tree that provides exactly that, with the same names and error classes.
"""

from __future__ import annotations

from collections.abc import Iterator, Mapping
from typing import Any, Union


class SymbolError(RuntimeError):
    """Base class of symbol errors (hc/symbols.py:24)."""


class SymbolConflictError(SymbolError):
    """A symbol was bound to two different values (hc/symbols.py:28)."""


class UnboundSymbolError(SymbolError):
    """An expression referenced a symbol with no value (hc/symbols.py:32)."""


class NonConstantError(SymbolError):
    """An expression could not be reduced to an integer (hc/symbols.py:40)."""


ExprLike = Union["Expr", int]


def _coerce(value: Any) -> Expr:
    if isinstance(value, Expr):
        return value
    if isinstance(value, bool):
        raise TypeError("bool is not an integer expression")
    if isinstance(value, int):
        return Const(value)
    try:
        import numpy as np

        if isinstance(value, np.integer):
            return Const(int(value))
    except ImportError:  # pragma: no cover - numpy is a hard dependency here
        pass
    raise TypeError(f"cannot use {type(value).__name__} as an integer expression")


def _floordiv(a: int, b: int) -> int:
    if b == 0:
        raise NonConstantError("division by zero in symbolic expression")
    return a // b


def _ceildiv(a: int, b: int) -> int:
    if b == 0:
        raise NonConstantError("division by zero in symbolic expression")
    return -((-a) // b)


def _mod(a: int, b: int) -> int:
    if b == 0:
        raise NonConstantError("modulo by zero in symbolic expression")
    return a % b


_OPS = {
    "+": (lambda a, b: a + b, "{} + {}"),
    "-": (lambda a, b: a - b, "{} - {}"),
    "*": (lambda a, b: a * b, "{} * {}"),
    "floor_div": (_floordiv, "floor_div({}, {})"),
    "ceil_div": (_ceildiv, "ceil_div({}, {})"),
    "mod": (_mod, "mod({}, {})"),
    "max": (max, "max({}, {})"),
    "min": (min, "min({}, {})"),
}


class Expr:
    """Integer expression over symbols."""

    __slots__ = ()

    def eval(self, env: Mapping[Any, int] | Env) -> int:  # noqa: A003 - reference name
        raise NotImplementedError

    def free_symbols(self) -> frozenset[Symbol]:
        raise NotImplementedError

    def _key(self) -> tuple:
        raise NotImplementedError

    def __eq__(self, other: object) -> bool:
        if isinstance(other, int) and not isinstance(other, bool):
            other = Const(other)
        if not isinstance(other, Expr):
            return NotImplemented
        return self._key() == other._key()

    def __hash__(self) -> int:
        return hash(self._key())

    def __add__(self, other: ExprLike) -> Expr:
        return BinOp("+", self, _coerce(other))

    def __radd__(self, other: ExprLike) -> Expr:
        return BinOp("+", _coerce(other), self)

    def __sub__(self, other: ExprLike) -> Expr:
        return BinOp("-", self, _coerce(other))

    def __rsub__(self, other: ExprLike) -> Expr:
        return BinOp("-", _coerce(other), self)

    def __mul__(self, other: ExprLike) -> Expr:
        return BinOp("*", self, _coerce(other))

    def __rmul__(self, other: ExprLike) -> Expr:
        return BinOp("*", _coerce(other), self)

    def __floordiv__(self, other: ExprLike) -> Expr:
        return BinOp("floor_div", self, _coerce(other))

    def __rfloordiv__(self, other: ExprLike) -> Expr:
        return BinOp("floor_div", _coerce(other), self)

    def __mod__(self, other: ExprLike) -> Expr:
        return BinOp("mod", self, _coerce(other))

    def __rmod__(self, other: ExprLike) -> Expr:
        return BinOp("mod", _coerce(other), self)

    def __neg__(self) -> Expr:
        return BinOp("-", Const(0), self)


class Const(Expr):
    __slots__ = ("value",)

    def __init__(self, value: int) -> None:
        self.value = int(value)

    def eval(self, env: Mapping[Any, int] | Env) -> int:  # noqa: A003
        return self.value

    def free_symbols(self) -> frozenset[Symbol]:
        return frozenset()

    def _key(self) -> tuple:
        return ("const", self.value)

    def __str__(self) -> str:
        return str(self.value)

    __repr__ = __str__


class Symbol(Expr):
    """A named integer symbol (``sym.M``)."""

    __slots__ = ("name",)

    def __init__(self, name: str) -> None:
        if not name or not name.isidentifier():
            raise ValueError(f"invalid symbol name {name!r}")
        self.name = name

    def eval(self, env: Mapping[Any, int] | Env) -> int:  # noqa: A003
        value = _lookup(env, self)
        if value is None:
            raise UnboundSymbolError(f"symbol {self.name} is unbound")
        return value

    def free_symbols(self) -> frozenset[Symbol]:
        return frozenset((self,))

    def _key(self) -> tuple:
        return ("sym", self.name)

    def __str__(self) -> str:
        return self.name

    __repr__ = __str__


class BinOp(Expr):
    __slots__ = ("op", "lhs", "rhs")

    def __init__(self, op: str, lhs: Expr, rhs: Expr) -> None:
        if op not in _OPS:
            raise ValueError(f"unknown operator {op}")
        self.op = op
        self.lhs = lhs
        self.rhs = rhs

    def eval(self, env: Mapping[Any, int] | Env) -> int:  # noqa: A003
        fn, _ = _OPS[self.op]
        return int(fn(self.lhs.eval(env), self.rhs.eval(env)))

    def free_symbols(self) -> frozenset[Symbol]:
        return self.lhs.free_symbols() | self.rhs.free_symbols()

    def _key(self) -> tuple:
        return ("op", self.op, self.lhs._key(), self.rhs._key())

    def __str__(self) -> str:
        _, fmt = _OPS[self.op]
        text = fmt.format(self.lhs, self.rhs)
        return f"({text})" if self.op in "+-*" else text

    __repr__ = __str__


def _lookup(env: Mapping[Any, int] | Env, symbol: Symbol) -> int | None:
    if isinstance(env, Env):
        return env.get(symbol)
    if symbol in env:
        return int(env[symbol])
    if symbol.name in env:
        return int(env[symbol.name])
    return None


class Env:
    """Immutable symbol -> integer environment (``Bindings.freeze()``)."""

    def __init__(self, values: Mapping[Symbol, int] | None = None) -> None:
        self._values: dict[Symbol, int] = dict(values or {})

    def get(self, symbol: Symbol) -> int | None:
        return self._values.get(symbol)

    def __getitem__(self, symbol: Symbol | str) -> int:
        key = sym_of(symbol) if isinstance(symbol, str) else symbol
        value = self._values.get(key)
        if value is None:
            raise UnboundSymbolError(f"symbol {key} is unbound")
        return value

    def __contains__(self, symbol: object) -> bool:
        if isinstance(symbol, str):
            symbol = sym_of(symbol)
        return symbol in self._values

    def __iter__(self) -> Iterator[Symbol]:
        return iter(self._values)

    def __len__(self) -> int:
        return len(self._values)

    def items(self):
        return self._values.items()

    def eval(self, expr: ExprLike) -> int:  # noqa: A003
        return _coerce(expr).eval(self)

    def __repr__(self) -> str:
        inner = ", ".join(f"{k}={v}" for k, v in self._values.items())
        return f"Env({inner})"


FrozenEnv = Env


class Bindings:
    """Mutable symbol bindings with conflict detection (hc/symbols.py:402-470)."""

    def __init__(self) -> None:
        self._bindings: dict[Symbol, int] = {}
        self._sources: dict[Symbol, str | None] = {}

    def bind(self, symbol: Symbol, value: int, *, source: str | None = None) -> None:
        value = int(value)
        existing = self._bindings.get(symbol)
        if existing is not None and existing != value:
            prev = self._sources.get(symbol)
            raise SymbolConflictError(
                f"conflicting binding for {symbol}: {existing} from {prev!r} vs "
                f"{value} from {source!r}"
            )
        self._bindings[symbol] = value
        self._sources[symbol] = source

    def bind_many(self, items: Mapping[Symbol, int], *, source: str | None = None) -> None:
        for symbol, value in items.items():
            self.bind(symbol, value, source=source)

    def require(self, expr: ExprLike, value: int, *, source: str | None = None) -> None:
        if isinstance(expr, bool):
            raise TypeError("require() does not accept bare bool values")
        node = _coerce(expr)
        actual = node.eval(self.freeze())
        if actual != int(value):
            raise SymbolConflictError(
                f"requirement failed at {source!r}: expected {node} == {value}, got {actual}"
            )

    def get(self, symbol: Symbol) -> int | None:
        return self._bindings.get(symbol)

    def freeze(self) -> Env:
        return Env(self._bindings)


_SYMBOLS: dict[str, Symbol] = {}


def sym_of(name: str) -> Symbol:
    symbol = _SYMBOLS.get(name)
    if symbol is None:
        symbol = Symbol(name)
        _SYMBOLS[name] = symbol
    return symbol


class _SymNamespace:
    """``sym.M`` returns the (interned) symbol named ``M``."""

    def __getattr__(self, name: str) -> Symbol:
        if name.startswith("__"):
            raise AttributeError(name)
        return sym_of(name)

    def __call__(self, name: str) -> Symbol:
        return sym_of(name)


sym = _SymNamespace()


def const(value: int) -> Expr:
    return Const(value)


def floor_div(a: ExprLike, b: ExprLike) -> Expr:
    return BinOp("floor_div", _coerce(a), _coerce(b))


def ceil_div(a: ExprLike, b: ExprLike) -> Expr:
    """ceil(a / b) for integers (hc/symbols.py:499-501)."""
    return BinOp("ceil_div", _coerce(a), _coerce(b))


def mod(a: ExprLike, b: ExprLike) -> Expr:
    return BinOp("mod", _coerce(a), _coerce(b))


def max_(a: ExprLike, b: ExprLike) -> Expr:
    return BinOp("max", _coerce(a), _coerce(b))


def min_(a: ExprLike, b: ExprLike) -> Expr:
    return BinOp("min", _coerce(a), _coerce(b))


__all__ = [
    "Bindings",
    "BinOp",
    "Const",
    "Env",
    "Expr",
    "FrozenEnv",
    "NonConstantError",
    "Symbol",
    "SymbolConflictError",
    "SymbolError",
    "UnboundSymbolError",
    "ceil_div",
    "const",
    "floor_div",
    "max_",
    "min_",
    "mod",
    "sym",
    "sym_of",
]
