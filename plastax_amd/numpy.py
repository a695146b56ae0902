"""jnp-style functions for writing device-traceable policies.

Import as ``import plastax_amd.numpy as jnp``. On traced values these build
expression nodes (see plastax_amd._expr); on plain numbers they compute in
float32 with numpy, so a policy also runs eagerly on host scalars.
"""

from __future__ import annotations

from typing import Any

import numpy as np

from plastax_amd._expr import (
    ConstArray,
    Expr,
    UnsupportedPolicyError,
    binary,
    cast,
    lift,
    select,
    unary,
    vector_sum,
)

float32 = np.float32
int32 = np.int32
uint32 = np.uint32
bool_ = np.bool_
inf = np.inf
nan = np.nan
pi = np.pi


def _traced(*xs: Any) -> bool:
    """Any operand traced: an expression, or an array holding expressions
    (a traced scalar broadcast against a constant array)."""
    return any(isinstance(x, Expr) or (isinstance(x, np.ndarray) and x.dtype == object) for x in xs)


def _unary(name: str, fn: Any) -> Any:
    def op(x: Any) -> Any:
        if _traced(x):
            return unary(name, x)
        return fn(np.float32(x))

    op.__name__ = name
    return op


tanh = _unary("tanh", np.tanh)
exp = _unary("exp", np.exp)
log = _unary("log", np.log)
sqrt = _unary("sqrt", np.sqrt)
cos = _unary("cos", np.cos)
sin = _unary("sin", np.sin)
log1p = _unary("log1p", np.log1p)
expm1 = _unary("expm1", np.expm1)
abs = _unary("abs", np.abs)  # noqa: A001 -- mirrors jnp.abs
absolute = abs
negative = _unary("neg", np.negative)
sign = _unary("sign", np.sign)


def square(x: Any) -> Any:
    if _traced(x):
        return unary("square", x)
    x = np.float32(x)
    return np.float32(x * x)


def _binary(name: str, fn: Any) -> Any:
    def op(a: Any, b: Any) -> Any:
        if _traced(a, b):
            return binary(name, a, b)
        return fn(np.float32(a), np.float32(b))

    op.__name__ = name
    return op


maximum = _binary("max", np.maximum)
minimum = _binary("min", np.minimum)
add = _binary("add", np.add)
subtract = _binary("sub", np.subtract)
multiply = _binary("mul", np.multiply)
divide = _binary("div", np.divide)
greater = _binary("gt", np.greater)
greater_equal = _binary("ge", np.greater_equal)
less = _binary("lt", np.less)
less_equal = _binary("le", np.less_equal)
equal = _binary("eq", np.equal)
not_equal = _binary("ne", np.not_equal)
floor = _unary("floor", np.floor)


def _int_binary(name: str, fn: Any) -> Any:
    def op(a: Any, b: Any) -> Any:
        if _traced(a, b):
            return binary(name, a, b)
        return fn(a, b)

    op.__name__ = name
    return op


floor_divide = _int_binary("floordiv", np.floor_divide)
remainder = _int_binary("mod", np.remainder)
mod = remainder
logical_and = _int_binary("and", np.logical_and)
logical_or = _int_binary("or", np.logical_or)
logical_xor = _int_binary("xor", np.logical_xor)
bitwise_and = _int_binary("and", np.bitwise_and)
bitwise_or = _int_binary("or", np.bitwise_or)
bitwise_xor = _int_binary("xor", np.bitwise_xor)
right_shift = _int_binary("shr", np.right_shift)
left_shift = _int_binary("shl", np.left_shift)


def logical_not(x: Any) -> Any:
    if _traced(x):
        return unary("not", cast(x, np.bool_))
    return np.logical_not(x)


def isfinite(x: Any) -> Any:
    """|x| < inf (false for NaN and the infinities)."""
    if _traced(x):
        return binary("lt", unary("abs", cast(x, np.float32)), np.float32(np.inf))
    return np.isfinite(x)


def astype(x: Any, dtype: Any) -> Any:
    if _traced(x):
        return cast(x, dtype)
    return np.asarray(x).astype(dtype)


def where(cond: Any, a: Any, b: Any) -> Any:
    if _traced(cond, a, b):
        return select(cond, a, b)
    return np.where(cond, np.float32(a), np.float32(b))


def sum(x: Any, axis: Any = None) -> Any:  # noqa: A001 -- mirrors jnp.sum
    """Sum over the traced output axis (a loss's reduction), or of a vector
    of traced scalars (e.g. ``jnp.sum(i >= starts)``: booleans count as
    int32)."""
    if isinstance(x, np.ndarray) and x.dtype == object:
        if axis not in (None, 0, -1):
            raise UnsupportedPolicyError("a traced vector sums over its one axis")
        return vector_sum(x)
    if _traced(x):
        if axis not in (None, 0, -1):
            raise UnsupportedPolicyError("traced sums reduce over the output axis only")
        return Expr("sum", (lift(x),))
    return np.sum(np.asarray(x, dtype=np.float32), axis=axis, dtype=np.float32)


def asarray(x: Any, dtype: Any = None) -> Any:
    """A traced value as is (cast to dtype); a constant as a ConstArray,
    which a traced policy may index with a traced integer."""
    if _traced(x):
        return x if dtype is None else cast(x, dtype)
    a = np.asarray(x, dtype=dtype)
    return a.view(ConstArray) if a.ndim >= 1 else a


def clip(x: Any, lo: Any, hi: Any) -> Any:
    return minimum(maximum(x, lo), hi)
