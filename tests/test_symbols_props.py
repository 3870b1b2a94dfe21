"""Properties of the symbolic integer expressions that size launches
(hc/symbols.py in the reference: ceil_div feeds work_shape), checked on
random trees and values: evaluation agrees with integer arithmetic, the
division identities hold, binding is consistent, and equal trees hash
equal.  CPU only."""

from __future__ import annotations

import pytest

hypothesis = pytest.importorskip("hypothesis")
from hypothesis import given, settings  # noqa: E402
from hypothesis import strategies as st  # noqa: E402

from hc.symbols import (  # noqa: E402
    Bindings,
    NonConstantError,
    SymbolConflictError,
    ceil_div,
    const,
    floor_div,
    max_,
    min_,
    mod,
    sym_of,
)

INTS = st.integers(min_value=-(1 << 40), max_value=1 << 40)
NONZERO = INTS.filter(lambda v: v != 0)
NAMES = ("M", "N", "K", "TILE")


@settings(max_examples=300, deadline=None)
@given(a=INTS, b=NONZERO)
def test_division_identities(a, b):
    q, r = floor_div(a, b).eval({}), mod(a, b).eval({})
    assert q * b + r == a
    assert abs(r) < abs(b) and (r == 0 or (r > 0) == (b > 0))
    c = ceil_div(a, b).eval({})
    if b > 0:
        # the smallest c with c * b >= a
        assert c * b >= a and (c - 1) * b < a
    assert c == q + (1 if r != 0 else 0)


OPS = ["+", "-", "*", "max", "min", "floor_div", "ceil_div", "mod"]


def _recipe(draw, depth):
    """A random expression tree as nested tuples: ("sym", name), ("const", v)
    or (op, lhs, rhs)."""
    if depth == 0 or draw(st.booleans()):
        if draw(st.booleans()):
            return ("sym", draw(st.sampled_from(NAMES)))
        return ("const", draw(st.integers(min_value=-50, max_value=50)))
    return (draw(st.sampled_from(OPS)), _recipe(draw, depth - 1), _recipe(draw, depth - 1))


def _build(recipe):
    kind = recipe[0]
    if kind == "sym":
        return sym_of(recipe[1])
    if kind == "const":
        return const(recipe[1])
    lhs, rhs = _build(recipe[1]), _build(recipe[2])
    return {"+": lambda: lhs + rhs, "-": lambda: lhs - rhs, "*": lambda: lhs * rhs,
            "max": lambda: max_(lhs, rhs), "min": lambda: min_(lhs, rhs),
            "floor_div": lambda: floor_div(lhs, rhs), "ceil_div": lambda: ceil_div(lhs, rhs),
            "mod": lambda: mod(lhs, rhs)}[kind]()


def _python(recipe, env):
    """The recipe evaluated with Python integers (ceil_div as -(-a // b))."""
    kind = recipe[0]
    if kind == "sym":
        return env[recipe[1]]
    if kind == "const":
        return recipe[1]
    a, b = _python(recipe[1], env), _python(recipe[2], env)
    return {"+": lambda: a + b, "-": lambda: a - b, "*": lambda: a * b, "max": lambda: max(a, b),
            "min": lambda: min(a, b), "floor_div": lambda: a // b, "ceil_div": lambda: -((-a) // b),
            "mod": lambda: a % b}[kind]()


@settings(max_examples=300, deadline=None)
@given(data=st.data())
def test_tree_evaluation_matches_integer_arithmetic(data):
    recipe = _recipe(data.draw, 4)
    values = {name: data.draw(st.integers(min_value=-1000, max_value=1000)) for name in NAMES}
    expr = _build(recipe)
    env = {sym_of(name): v for name, v in values.items()}
    try:
        want = _python(recipe, values)
    except ZeroDivisionError:
        with pytest.raises(NonConstantError):
            expr.eval(env)
        return
    assert expr.eval(env) == want


@settings(max_examples=200, deadline=None)
@given(data=st.data())
def test_equal_trees_are_equal_and_hash_equal(data):
    recipe = _recipe(data.draw, 3)
    a, b = _build(recipe), _build(recipe)
    assert a == b and hash(a) == hash(b) and str(a) == str(b)
    assert a.free_symbols() == frozenset(sym_of(n) for n in NAMES if ("sym", n) in _leaves(recipe))


def _leaves(recipe):
    if recipe[0] in ("sym", "const"):
        return {recipe}
    return _leaves(recipe[1]) | _leaves(recipe[2])


@settings(max_examples=200, deadline=None)
@given(m=st.integers(min_value=0, max_value=1 << 20), other=st.integers(min_value=0, max_value=1 << 20))
def test_binding_is_idempotent_and_conflicts_are_reported(m, other):
    b = Bindings()
    b.bind(sym_of("M"), m)
    b.bind(sym_of("M"), m)  # the same value again is accepted
    assert b.get(sym_of("M")) == m
    b.require(ceil_div(sym_of("M"), 16), -((-m) // 16))
    if other != m:
        with pytest.raises(SymbolConflictError):
            b.bind(sym_of("M"), other)
