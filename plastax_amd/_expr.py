"""Symbolic tracing of user policies into device unit programs.

The reference traces every policy callback with JAX and lowers the jaxpr
(phases.py:535-556 reads ``linear_input``; phases.py:1910-2147 translates
prune predicates to Triton source). This module plays the same role for the
device library: a policy's ``map`` / ``apply`` / ``calculate_loss`` is called
once with symbolic views, the returned expression tree is checked against what
the kernels run, and an ``apply`` or an elementwise loss is compiled to a
register program that the kernels interpret per unit (``plx_program`` in
include/plastax_hip.h). The program keeps the user's float32 operation order,
so a traced apply rounds exactly as the reference's jnp expression does.

User policies write jnp-style code against :mod:`plastax_amd.numpy` (``jnp``)
and :mod:`plastax_amd.nn`; anything the tracer cannot represent raises
:class:`UnsupportedPolicyError` when the step is built.
"""

from __future__ import annotations

import dataclasses
from typing import Any, Iterable, Sequence

import numpy as np

from plastax_amd._types import FieldSpec


class UnsupportedPolicyError(NotImplementedError):
    """A policy the device path cannot run (raised when a step is built)."""


class TracerBoolError(UnsupportedPolicyError):
    """Python control flow on a traced value (use jnp.where instead)."""


# Opcodes: keep in sync with plastax_amd/csrc/plastax_hip.hip (and the
# oracle's evaluator).
OPCODES = {
    "acc": 1,
    "ldu": 2,
    "const": 3,
    "add": 4,
    "sub": 5,
    "mul": 6,
    "div": 7,
    "neg": 8,
    "abs": 9,
    "max": 10,
    "min": 11,
    "tanh": 12,
    "exp": 13,
    "log": 14,
    "sqrt": 15,
    "sigmoid": 16,
    "gt": 17,
    "ge": 18,
    "lt": 19,
    "le": 20,
    "eq": 21,
    "ne": 22,
    "sel": 23,
    "out": 24,
    "target": 25,
    "mov": 26,
    "square": 27,
    "relu": 28,
    "sign": 29,
    "log1p": 30,
    "expm1": 31,
    "cos": 33,
    "sin": 34,
}
_UNARY = {"neg", "abs", "tanh", "exp", "log", "sqrt", "sigmoid", "square", "relu", "sign", "cos", "sin", "log1p",
          "expm1"}
_BINARY = {"add", "sub", "mul", "div", "max", "min", "gt", "ge", "lt", "le", "eq", "ne"}
MAX_REGS = 16
MAX_INSTR = 48
MAX_CONST = 32
MAX_FIELDS = 8
MAX_OUTS = 4


def _f32(x: Any) -> np.float32:
    return np.float32(x)


# Value kinds of a traced expression: float32 ("f"), int32 ("i"), uint32
# ("u"), bool ("b"), and the weakly typed Python scalars ("wi", "wf") that
# take the other operand's type, as jnp's weak typing does.
_WEAK = {"wi", "wf"}
_FLOAT_ONLY = {"tanh", "exp", "log", "sqrt", "sigmoid", "floor", "cos", "sin", "log1p", "expm1"}
_INT_ONLY = {"mod", "floordiv", "shl", "shr"}
_LOGIC = {"and", "or", "xor"}


def kind_of_dtype(dtype: Any) -> str:
    """The value kind of a numpy dtype (x64 off: 64-bit types narrow to 32)."""
    dt = np.dtype(dtype)
    if dt == np.bool_:
        return "b"
    if dt.kind == "f":
        return "f"
    if dt.kind == "u":
        return "u"
    if dt.kind == "i":
        return "i"
    raise UnsupportedPolicyError(f"dtype {dt} cannot be traced")


def _promote(a: "Expr", b: "Expr", op: str) -> str:
    """The result kind of a binary arithmetic op (jnp promotion, x64 off)."""
    ka, kb = a.dtype, b.dtype
    strong = {k for k in (ka, kb) if k not in _WEAK}
    weak = {k for k in (ka, kb) if k in _WEAK}
    if not strong:
        return "wf" if "wf" in weak else "wi"
    if "f" in strong:
        return "f"
    if "i" in strong and "u" in strong:
        raise UnsupportedPolicyError("int32 mixed with uint32 promotes to 64 bits in jnp")
    if "wf" in weak:
        return "f"
    if "i" in strong:
        return "i"
    if "u" in strong:
        return "u"
    # only bools
    if weak:
        return "i"
    if op in _LOGIC or op in ("eq", "ne", "max", "min"):
        return "b"
    raise UnsupportedPolicyError(f"arithmetic {op!r} on two booleans")


def _as_kind(x: "Expr", kind: str) -> "Expr":
    """``x`` as a value of ``kind`` (constants are retyped, others cast)."""
    if x.dtype == kind:
        return x
    if x.op == "const":
        return Expr("const", value=x.value, dtype=kind)
    return Expr("cvt", (x,), dtype=kind)


def _is_vector(x: Any) -> bool:
    return isinstance(x, np.ndarray) and x.ndim == 1


def _elements(x: Any, n: int) -> list:
    if _is_vector(x):
        if x.size != n:
            raise UnsupportedPolicyError(f"constant arrays of lengths {x.size} and {n} do not broadcast")
        return [x[k] for k in range(n)]
    return [x] * n


def vector_binary(op: str, a: Any, b: Any) -> np.ndarray:
    """An elementwise op where an operand is a 1-D constant array (or an
    array of traced values): an object array of traced scalars, one per
    element (jnp broadcasting of a scalar against a vector)."""
    n = a.size if _is_vector(a) else b.size
    out = np.empty(n, dtype=object)
    for k, (x, y) in enumerate(zip(_elements(a, n), _elements(b, n))):
        out[k] = binary(op, x, y)
    return out


def const_gather(values: np.ndarray, key: Any) -> "Expr":
    """``values[key]`` for a 1-D constant array and a traced integer, with
    jnp's gather semantics: a negative index counts from the end, then the
    index is clamped into the array (an out-of-range read returns the
    nearest end). Compiled as a chain of selects."""
    values = np.asarray(values)
    if values.ndim != 1 or values.size == 0:
        raise UnsupportedPolicyError("a traced index reads a non-empty 1-D constant array")
    k = lift(key)
    if k.dtype in ("f", "wf", "b"):
        raise UnsupportedPolicyError("an array index must be an integer")
    n = values.size
    k = select(binary("lt", k, 0), binary("add", k, n), k)
    out: Any = values[n - 1]
    for j in range(n - 2, -1, -1):
        out = select(binary("le", k, j), values[j], out)
    return lift(out)


def vector_sum(x: np.ndarray) -> "Expr":
    """jnp.sum of a vector of traced scalars: booleans count as int32; the
    elements fold left to right (a float sum over a constant-length vector
    rounds in that order)."""
    items = [lift(v) for v in x]
    if not items:
        return Expr("const", value=0, dtype="wi")
    items = [_as_kind(v, "i") if v.dtype == "b" else v for v in items]
    out = items[0]
    for v in items[1:]:
        out = binary("add", out, v)
    return out


class ConstArray(np.ndarray):
    """A constant array a traced policy may index with a traced integer
    (``table[layer]``, see const_gather) or compare and combine with traced
    scalars elementwise; on concrete indices it is a plain numpy array.
    ``plastax_amd.numpy.asarray`` returns one for non-traced input."""

    def __getitem__(self, key: Any) -> Any:
        if isinstance(key, Expr):
            return const_gather(self.view(np.ndarray), key)
        return super().__getitem__(key)


def binary(op: str, a: Any, b: Any) -> "Expr":
    """A typed binary node: arithmetic, comparison or logical."""
    if _is_vector(a) or _is_vector(b):
        return vector_binary(op, a, b)  # type: ignore[return-value]
    a, b = lift(a), lift(b)
    if op == "div":
        t = "f"  # true division: ints go to float32, as jnp's / does
    else:
        t = _promote(a, b, op)
    if t in _WEAK:
        t = "f" if t == "wf" else "i"
    if op in _INT_ONLY and t not in ("i", "u"):
        raise UnsupportedPolicyError(f"{op!r} is traced on integers only")
    if op in _LOGIC and t not in ("b", "i", "u"):
        raise UnsupportedPolicyError(f"{op!r} is traced on booleans and integers only")
    a2, b2 = _as_kind(a, t), _as_kind(b, t)
    out = "b" if op in ("gt", "ge", "lt", "le", "eq", "ne") else t
    return Expr(op, (a2, b2), dtype=out)


def unary(op: str, x: Any) -> "Expr":
    """A typed unary node."""
    x = lift(x)
    k = x.dtype
    if k in _WEAK:
        k = "f" if k == "wf" else "i"
    if op in _FLOAT_ONLY or k == "b" and op not in ("not",):
        k = "f"
    if op == "not":
        if k not in ("b", "i", "u"):
            raise UnsupportedPolicyError("~ is traced on booleans and integers only")
    return Expr(op, (_as_kind(x, k),), dtype=k)


def select(cond: Any, a: Any, b: Any) -> "Expr":
    """where(cond, a, b): the branches promoted to one kind."""
    c = lift(cond)
    if c.dtype != "b":
        c = binary("ne", c, Expr("const", value=0, dtype="wi"))
    a, b = lift(a), lift(b)
    t = _promote(a, b, "sel")
    if t in _WEAK:
        t = "f" if t == "wf" else "i"
    return Expr("sel", (c, _as_kind(a, t), _as_kind(b, t)), dtype=t)


def cast(x: Any, dtype: Any) -> "Expr":
    """x.astype(dtype)."""
    x = lift(x)
    k = kind_of_dtype(dtype)
    return _as_kind(x, k)


class Expr:
    """A node of a traced expression; ``dtype`` is its value kind."""

    __slots__ = ("op", "args", "value", "field", "role", "dtype")
    __array_ufunc__ = None  # numpy scalars defer to the reflected operators

    def __init__(
        self,
        op: str,
        args: Sequence["Expr"] = (),
        *,
        value: Any = None,
        field: str | None = None,
        role: str | None = None,
        dtype: str = "f",
    ) -> None:
        self.op = op
        self.args = tuple(args)
        self.value = value
        self.field = field
        self.role = role
        self.dtype = dtype

    # -- construction helpers -------------------------------------------------
    def __repr__(self) -> str:
        if self.op == "const":
            return repr(self.value)
        if self.op in ("ldu", "ldc"):
            return f"{self.field}[{self.role}]"
        if self.op in ("acc", "target", "global"):
            return self.op if self.field is None else f"g.{self.field}"
        if self.op == "idx":
            return str(self.role)
        return f"{self.op}({', '.join(map(repr, self.args))})"

    def __bool__(self) -> bool:
        raise TracerBoolError(
            "a traced policy value was used in Python control flow; use jnp.where"
        )

    __hash__ = object.__hash__

    # -- arithmetic -----------------------------------------------------------
    def __add__(self, o: Any) -> "Expr":
        return binary("add", self, o)

    def __radd__(self, o: Any) -> "Expr":
        return binary("add", o, self)

    def __sub__(self, o: Any) -> "Expr":
        return binary("sub", self, o)

    def __rsub__(self, o: Any) -> "Expr":
        return binary("sub", o, self)

    def __mul__(self, o: Any) -> "Expr":
        return binary("mul", self, o)

    def __rmul__(self, o: Any) -> "Expr":
        return binary("mul", o, self)

    def __truediv__(self, o: Any) -> "Expr":
        return binary("div", self, o)

    def __rtruediv__(self, o: Any) -> "Expr":
        return binary("div", o, self)

    def __floordiv__(self, o: Any) -> "Expr":
        return binary("floordiv", self, o)

    def __rfloordiv__(self, o: Any) -> "Expr":
        return binary("floordiv", o, self)

    def __mod__(self, o: Any) -> "Expr":
        return binary("mod", self, o)

    def __rmod__(self, o: Any) -> "Expr":
        return binary("mod", o, self)

    def __lshift__(self, o: Any) -> "Expr":
        return binary("shl", self, o)

    def __rshift__(self, o: Any) -> "Expr":
        return binary("shr", self, o)

    def __and__(self, o: Any) -> "Expr":
        return binary("and", self, o)

    def __rand__(self, o: Any) -> "Expr":
        return binary("and", o, self)

    def __or__(self, o: Any) -> "Expr":
        return binary("or", self, o)

    def __ror__(self, o: Any) -> "Expr":
        return binary("or", o, self)

    def __xor__(self, o: Any) -> "Expr":
        return binary("xor", self, o)

    def __rxor__(self, o: Any) -> "Expr":
        return binary("xor", o, self)

    def __invert__(self) -> "Expr":
        return unary("not", self)

    def __neg__(self) -> "Expr":
        return unary("neg", self)

    def __pos__(self) -> "Expr":
        return self

    def __abs__(self) -> "Expr":
        return unary("abs", self)

    def __pow__(self, o: Any) -> "Expr":
        # jnp's x ** 2 lowers to integer_pow, i.e. one multiply x * x.
        if isinstance(o, (int, np.integer)) and int(o) == 2:
            return unary("square", self)
        if isinstance(o, (int, np.integer)) and int(o) == 1:
            return self
        raise UnsupportedPolicyError(f"only x ** 2 is supported in a traced policy, got ** {o!r}")

    def __gt__(self, o: Any) -> "Expr":
        return binary("gt", self, o)

    def __ge__(self, o: Any) -> "Expr":
        return binary("ge", self, o)

    def __lt__(self, o: Any) -> "Expr":
        return binary("lt", self, o)

    def __le__(self, o: Any) -> "Expr":
        return binary("le", self, o)

    def __eq__(self, o: Any) -> "Expr":  # type: ignore[override]
        return binary("eq", self, o)

    def __ne__(self, o: Any) -> "Expr":  # type: ignore[override]
        return binary("ne", self, o)

    def astype(self, dtype: Any) -> "Expr":
        return cast(self, dtype)


def lift(x: Any) -> Expr:
    """A traced value, or a constant node for a Python/numpy scalar (Python
    scalars are weakly typed; numpy scalars carry their dtype)."""
    if isinstance(x, Expr):
        return x
    if isinstance(x, (bool, np.bool_)):
        return Expr("const", value=bool(x), dtype="b")
    if isinstance(x, int):
        return Expr("const", value=int(x), dtype="wi")
    if isinstance(x, float):
        return Expr("const", value=float(x), dtype="wf")
    if isinstance(x, (np.integer, np.floating)):
        return Expr("const", value=x.item(), dtype=kind_of_dtype(x.dtype))
    if isinstance(x, np.ndarray) and x.shape == ():
        return Expr("const", value=x.item(), dtype=kind_of_dtype(x.dtype))
    raise UnsupportedPolicyError(f"cannot trace a {type(x).__name__} value in a policy")


# ---------------------------------------------------------------------------
# Symbolic views handed to policies while tracing.
# ---------------------------------------------------------------------------


@dataclasses.dataclass(frozen=True)
class Index:
    """A symbolic unit/connection index (the role it plays for the edge)."""

    role: str  # "self", "src", "dst", "out", "cid"


class TraceUnitView:
    """Symbolic stand-in for views.UnitView: ``u[FIELD, idx]``."""

    def __init__(self, dtypes: dict[str, np.dtype]) -> None:
        self._dtypes = dtypes

    def _load(self, spec: FieldSpec, role: str) -> Expr:
        name = spec.name
        if name not in self._dtypes:
            raise UnsupportedPolicyError(f"unit field {name!r} is not a column of this net")
        return Expr("ldu", field=name, role=role)

    def __getitem__(self, key: tuple[FieldSpec, Any]) -> Expr:
        spec, idx = key
        if isinstance(idx, Index):
            return self._load(spec, idx.role)
        if isinstance(idx, Expr) and idx.op == "ldc" and idx.field in ("from_id", "to_id"):
            return self._load(spec, "src" if idx.field == "from_id" else "dst")
        fixed = _fixed_index(idx)
        if fixed is not None:
            e = self._load(spec, "fixed")
            e.value = fixed
            return e
        raise UnsupportedPolicyError(f"unit field read at an untraceable index {idx!r}")

    def gather(self, spec: FieldSpec, ids: Any) -> Expr:
        if isinstance(ids, Index):
            return self._load(spec, ids.role)
        raise UnsupportedPolicyError("UnitView.gather is traced only over the output ids")


def _fixed_index(idx: Any) -> int | None:
    """A unit index known at trace time (``UnitIdx(jnp.int32(k))``), or None."""
    if isinstance(idx, (bool, np.bool_)):
        return None
    if isinstance(idx, (int, np.integer)):
        return int(idx)
    if isinstance(idx, np.ndarray) and idx.shape == () and np.issubdtype(idx.dtype, np.integer):
        return int(idx)
    return None


class TraceConnView:
    """Symbolic stand-in for views.ConnView: ``c[FIELD, cid]``."""

    def __init__(self, dtypes: dict[str, np.dtype]) -> None:
        self._dtypes = dtypes

    def __getitem__(self, key: tuple[FieldSpec, Any]) -> Expr:
        spec, idx = key
        if not (isinstance(idx, Index) and idx.role == "cid"):
            raise UnsupportedPolicyError("connection fields are read at the edge's own cid")
        if spec.name not in self._dtypes:
            raise UnsupportedPolicyError(f"conn field {spec.name!r} is not a column of this net")
        return Expr("ldc", field=spec.name, role="cid")


class TraceGlobals:
    """Symbolic globals: ``g["name"]`` / ``g.name`` read a scalar global."""

    def __init__(self, concrete: Any) -> None:
        self._concrete = concrete

    def __getitem__(self, key: str) -> Expr:
        return Expr("global", field=str(key))

    def __getattr__(self, key: str) -> Expr:
        if key.startswith("_"):
            raise AttributeError(key)
        return Expr("global", field=key)


# ---------------------------------------------------------------------------
# Pattern checks for the per-edge map.
# ---------------------------------------------------------------------------


@dataclasses.dataclass(frozen=True)
class ProductMap:
    """A traced map of the product form (connection factor) * (unit factor
    at the edge's other end). ``field`` is the unit field gathered at the
    other end (None: the constant ``x_const``); the connection factor is
    WEIGHT unless ``w_const`` is set. A lone factor is its product with 1.0,
    which leaves every float32 bit unchanged."""

    field: str | None
    w_const: np.float32 | None = None
    x_const: np.float32 | None = None


def _float_const(x: Any) -> np.float32 | None:
    if isinstance(x, Expr) and x.op == "const" and x.dtype in ("f", "wf", "wi"):
        return np.float32(x.value)
    return None


def product_map(expr: Any, other_role: str) -> ProductMap:
    """The factors of a map the device runs: ``c[WEIGHT, cid] * u[F, other]``
    (the reference's ``linear_input`` contract, phases.py:535-556; either
    operand order, as float multiplication commutes bit for bit), either
    factor replaced by a float constant, or a lone factor (``c[WEIGHT, cid]``,
    ``u[F, other]`` or a constant, e.g. 1.0 to count the live edges)."""

    def factor(x: Any) -> tuple[str, Any] | None:
        if isinstance(x, Expr) and x.op == "ldc" and x.field == "weight":
            return ("w", None)
        if isinstance(x, Expr) and x.op == "ldu" and x.role == other_role and x.dtype == "f":
            return ("x", str(x.field))
        k = _float_const(x)
        return None if k is None else ("k", k)

    expr = lift(expr)
    if isinstance(expr, Expr) and expr.op == "mul":
        parts = [factor(x) for x in expr.args]
    else:
        parts = [factor(expr), ("k", np.float32(1.0))]
    if all(p is not None for p in parts):
        ws = [v for k, v in parts if k == "w"]
        xs = [v for k, v in parts if k == "x"]
        ks = [v for k, v in parts if k == "k"]
        if len(ws) <= 1 and len(xs) <= 1:
            w_const = None if ws else ks.pop(0)
            return ProductMap(xs[0] if xs else None, w_const, None if xs else ks.pop(0))
    raise UnsupportedPolicyError(
        f"map must be c[WEIGHT, cid] * u[FIELD, {other_role}] (either factor may be a float "
        f"constant, or stand alone) to run on the device, got {expr!r}"
    )


def linear_map_field(expr: Any, other_role: str) -> str:
    """The unit field a map multiplies the edge weight by (the linear form
    ``c[WEIGHT, cid] * u[F, other]``; see product_map for the general one)."""
    pm = product_map(expr, other_role)
    if pm.field is None or pm.w_const is not None or pm.x_const is not None:
        raise UnsupportedPolicyError(
            f"map must be c[WEIGHT, cid] * u[FIELD, {other_role}] here, got {expr!r}"
        )
    return pm.field


# ---------------------------------------------------------------------------
# Program compilation.
# ---------------------------------------------------------------------------


@dataclasses.dataclass
class Program:
    """A compiled unit program (plx_program)."""

    code: list[tuple[int, int, int, int]]
    consts: list[np.float32]
    fields: list[str]  # LDU operand table (unit field names)
    out_fields: list[str | None]  # OUT slot -> unit field written (None: returned)
    globals_at: dict[int, str]  # const slot -> global name, refreshed per call
    # LDU operand slot -> the one unit it is read at (a loss reading a unit
    # fixed at trace time, e.g. u[F, UnitIdx(k)]); other slots read the
    # program's own unit.
    fixed_at: dict[int, int] = dataclasses.field(default_factory=dict)

    @property
    def ninstr(self) -> int:
        return len(self.code)

    def flat_code(self) -> np.ndarray:
        return np.asarray(self.code, dtype=np.int32).reshape(-1)

    def const_values(self, globals_: Any = None) -> np.ndarray:
        vals = np.asarray(self.consts, dtype=np.float32).copy()
        for slot, name in self.globals_at.items():
            vals[slot] = np.float32(_read_global(globals_, name))
        return vals


def _read_global(g: Any, name: str) -> Any:
    if isinstance(g, dict):
        v = g[name]
    else:
        v = getattr(g, name)
    arr = np.asarray(v)
    if arr.shape != ():
        raise UnsupportedPolicyError(f"global {name!r} must be a scalar to be traced")
    return arr


def compile_program(
    outputs: Sequence[Any], out_fields: Sequence[str | None], *, allow: Iterable[str]
) -> Program:
    """Compile expression outputs to a register program.

    ``allow`` names the leaf kinds the context permits: "acc" (apply),
    "target" (loss), and the unit-field roles ("self" or "out", and "fixed":
    a unit index known at trace time).
    """
    allowed = set(allow)
    outs = [lift(o) for o in outputs]
    if len(outs) > MAX_OUTS:
        raise UnsupportedPolicyError(f"a policy writes {len(outs)} fields; at most {MAX_OUTS}")

    order: list[Expr] = []
    seen: set[int] = set()

    def visit(e: Expr) -> None:
        stack = [(e, False)]
        while stack:
            node, done = stack.pop()
            if id(node) in seen:
                continue
            if done:
                seen.add(id(node))
                order.append(node)
                continue
            stack.append((node, True))
            for a in reversed(node.args):
                if id(a) not in seen:
                    stack.append((a, False))

    for o in outs:
        visit(o)

    # Last use of each node, for register reuse.
    last_use: dict[int, int] = {}
    for pos, node in enumerate(order):
        for a in node.args:
            last_use[id(a)] = pos
    for o in outs:
        last_use[id(o)] = len(order)

    consts: list[np.float32] = []
    const_slot: dict[Any, int] = {}
    globals_at: dict[int, str] = {}
    fields: list[str] = []
    field_slot: dict[tuple[str, int | None], int] = {}
    fixed_at: dict[int, int] = {}
    reg: dict[int, int] = {}
    free = list(range(MAX_REGS - 1, -1, -1))
    code: list[tuple[int, int, int, int]] = []

    def const_index(key: Any, value: np.float32) -> int:
        if key not in const_slot:
            if len(consts) >= MAX_CONST:
                raise UnsupportedPolicyError("a policy uses too many constants")
            const_slot[key] = len(consts)
            consts.append(value)
        return const_slot[key]

    for pos, node in enumerate(order):
        if not free:
            raise UnsupportedPolicyError("a policy expression needs too many registers")
        op = node.op
        if node.dtype in ("i", "u") and op != "const":
            raise UnsupportedPolicyError(
                f"integer arithmetic ({op!r}) cannot run in a unit program"
            )
        if op == "const":
            k = const_index(("c", np.float32(node.value).tobytes()), np.float32(node.value))
            instr = ("const", k, 0)
        elif op == "cvt":
            if node.args[0].dtype not in ("f", "b", "wf", "wi"):
                raise UnsupportedPolicyError("integer casts cannot run in a unit program")
            instr = ("mov", reg[id(node.args[0])], 0)
        elif op == "global":
            k = const_index(("g", node.field), np.float32(0.0))
            globals_at[k] = str(node.field)
            instr = ("const", k, 0)
        elif op == "acc":
            if "acc" not in allowed:
                raise UnsupportedPolicyError("the accumulator is only visible to apply")
            instr = ("acc", 0, 0)
        elif op == "target":
            if "target" not in allowed:
                raise UnsupportedPolicyError("targets are only visible to the loss")
            instr = ("target", 0, 0)
        elif op == "ldu":
            if node.role not in allowed:
                where = "a fixed unit" if node.role == "fixed" else repr(node.role)
                raise UnsupportedPolicyError(
                    f"unit field {node.field!r} read at {where}: only the unit's own "
                    "fields are visible here"
                )
            key = (str(node.field), int(node.value) if node.role == "fixed" else None)
            if key not in field_slot:
                if len(fields) >= MAX_FIELDS:
                    raise UnsupportedPolicyError("a policy reads too many unit fields")
                field_slot[key] = len(fields)
                fields.append(key[0])
                if key[1] is not None:
                    if key[1] < 0:
                        raise UnsupportedPolicyError(f"unit index {key[1]} is negative")
                    fixed_at[field_slot[key]] = key[1]
            instr = ("ldu", field_slot[key], 0)
        elif op in _UNARY:
            instr = (op, reg[id(node.args[0])], 0)
        elif op in _BINARY:
            instr = (op, reg[id(node.args[0])], reg[id(node.args[1])])
        elif op == "sel":
            # r[d] = r[a] != 0 ? r[b] : r[b+1]: the two branches go to a
            # consecutive register pair.
            c, t, f = (reg[id(a)] for a in node.args)
            if not free or len(free) < 2:
                raise UnsupportedPolicyError("a policy expression needs too many registers")
            pair = _take_pair(free)
            code.append((OPCODES["mov"], pair, t, 0))
            code.append((OPCODES["mov"], pair + 1, f, 0))
            instr = ("sel", c, pair)
        elif op == "ldc":
            raise UnsupportedPolicyError("connection fields are not visible to a unit program")
        else:
            raise UnsupportedPolicyError(f"operation {op!r} cannot run on the device")
        # Release operands whose last use is here before picking a register.
        for a in node.args:
            if last_use.get(id(a)) == pos and reg[id(a)] not in free:
                free.append(reg[id(a)])
        d = free.pop()
        reg[id(node)] = d
        name, a0, b0 = instr
        code.append((OPCODES[name], d, a0, b0))
        if op == "sel":
            free.append(b0)
            free.append(b0 + 1)
    for slot, o in enumerate(outs):
        code.append((OPCODES["out"], slot, reg[id(o)], 0))
    if len(code) > MAX_INSTR:
        raise UnsupportedPolicyError(f"a policy compiles to {len(code)} instructions; at most {MAX_INSTR}")
    return Program(code, consts, fields, list(out_fields), globals_at, fixed_at)


def _take_pair(free: list[int]) -> int:
    s = set(free)
    for r in range(0, MAX_REGS - 1):
        if r in s and r + 1 in s:
            free.remove(r)
            free.remove(r + 1)
            return r
    raise UnsupportedPolicyError("a policy expression needs too many registers")
