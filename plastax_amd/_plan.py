"""Trace a Network's policies into the device plan of its step.

``build_phases`` (phases.py:87-182) decides the reference's phase tuple at
trace time; ``compile_plan`` makes the same decisions for the device and
checks that every present policy has a device lowering:

- forward / backward: the map must be of the product form
  ``WEIGHT * field[other]`` (the ``linear_input`` contract of
  phases.py:535-556), either factor possibly a float constant or absent
  (``_expr.product_map``: a constant map counts live edges), the combine a
  named monoid, and ``apply`` is compiled to a unit program;
- loss: ``SoftmaxCrossEntropyLoss`` runs its own kernel; any other loss must
  return ``(jnp.sum(term), seed)`` with ``term`` and ``seed`` elementwise in
  the output's prediction and target, and is compiled to a program;
- update_conn: one of the optim bundles (fused update kernel), or any other
  UpdateConn, whose ``incoming`` / ``outgoing`` run as edge site programs
  (``update_generic``; traced when the step first runs, against its globals).

Policies outside these forms raise UnsupportedPolicyError.
"""

from __future__ import annotations

import dataclasses
from typing import Any

import numpy as np

from plastax_amd import _lib
from plastax_amd._expr import (
    Expr,
    Index,
    Program,
    TraceConnView,
    TraceGlobals,
    TraceUnitView,
    UnsupportedPolicyError,
    compile_program,
    product_map,
)
from plastax_amd.growth_config import GrowthConfig
from plastax_amd.monoid import Monoid
from plastax_amd.optim._rules import _RuleBase
from plastax_amd.state import NetworkStatic
from plastax_amd.traits import SoftmaxCrossEntropyLoss
from plastax_amd.views import UnitWrite

POW_TABLE_LEN = 1 << 16


@dataclasses.dataclass
class GenericPass:
    """A pass outside the product form: any map (one float32 component, or a
    tuple with a tuple of monoids), folded per row by the map's edge program
    and applied by a unit program (traced on the step's first call, against
    its globals)."""

    policy: Any
    backward: bool
    monoids: tuple[int, ...]  # PLX_MONOID_* per component
    identities: tuple[float, ...]
    tuple_acc: bool
    why: str  # why the product form did not apply


@dataclasses.dataclass
class PassPlan:
    """A traced forward or backward pass."""

    field: str | None  # the unit field the map gathers at the other end (None: x_const)
    monoid: int
    identity: float
    program: Program  # the apply
    w_const: np.float32 | None = None  # the map's connection factor, when not WEIGHT
    x_const: np.float32 | None = None  # the map's unit factor, when not a field
    generic: GenericPass | None = None  # set: the pass runs as edge / unit programs

    def map_struct(self) -> "_lib.plx_map":
        """The plx_map of this pass's map."""
        m = _lib.plx_map()
        if self.w_const is not None:
            m.flags |= _lib.PLX_MAP_W_CONST
            m.w = float(self.w_const)
        if self.x_const is not None:
            m.flags |= _lib.PLX_MAP_X_CONST
            m.x = float(self.x_const)
        return m

    def gathered(self, units: dict, fallback: str) -> Any:
        """The unit column the kernels gather for the map: the field, or
        (for a constant unit factor, never read for the term) ``fallback``."""
        return units[self.field if self.field is not None else fallback]


@dataclasses.dataclass
class LossPlan:
    kind: str  # "softmax" or "elementwise"
    seed_field: str
    program: Program | None = None


@dataclasses.dataclass
class Plan:
    forward: PassPlan
    loss: LossPlan | None
    backward: PassPlan | None
    update: Any  # an optim _RuleBase or None
    net: Any = None  # the Network class (its unit / structural policies are traced lazily)
    update_unit: bool = False
    prune_unit: bool = False
    prune_conn: bool = False
    add_unit: bool = False
    add_conn: Any = None  # the validated GrowthConfig, or None
    reset_global: bool = False
    update_generic: bool = False  # update_conn is a user UpdateConn (edge programs)

    def pow_table(self) -> np.ndarray:
        """float32(b1^t), float32(b2^t) for t < POW_TABLE_LEN, by binary
        exponentiation in float64 (the device's pow_step, bit for bit)."""
        p = self.update.params()
        b1, b2 = float(p[1]), float(p[2])
        t = np.arange(POW_TABLE_LEN, dtype=np.int64)
        out = np.empty((POW_TABLE_LEN, 2), dtype=np.float32)
        for col, b in enumerate((b1, b2)):
            acc = np.ones(POW_TABLE_LEN, dtype=np.float64)
            base = np.float64(b)
            n = t.copy()
            while bool(n.any()):
                odd = (n & 1).astype(bool)
                acc = np.where(odd, acc * base, acc)
                base = base * base
                n >>= 1
            out[:, col] = acc.astype(np.float32)
        return out.reshape(-1)


def _float_unit_fields(static: NetworkStatic) -> dict[str, np.dtype]:
    return {s.name: np.dtype(s.dtype) for s in static.unit_fields}


def _check_float_fields(names: list[str | None], dtypes: dict[str, np.dtype], what: str) -> None:
    for name in names:
        if name is None:
            continue
        if name not in dtypes:
            raise UnsupportedPolicyError(f"{what} writes {name!r}, which is not a unit column")
        if dtypes[name] != np.float32:
            raise UnsupportedPolicyError(f"{what} touches {name!r}, which is not float32")


def _generic_pass(policy: Any, *, backward: bool, why: str) -> PassPlan:
    """The plan of a pass whose map is not of the product form."""
    name = type(policy).__name__
    combine = policy.combine
    monoids = combine if isinstance(combine, tuple) else (combine,)
    if not monoids or not all(isinstance(m, Monoid) for m in monoids):
        raise UnsupportedPolicyError(f"{name}.combine must be a named monoid or a tuple of them")
    if len(monoids) > 8:
        raise UnsupportedPolicyError(f"{name}: at most 8 accumulator components")
    codes = tuple(m.code for m in monoids)
    idents = tuple(float(m.identity_for()) for m in monoids)
    gp = GenericPass(policy, backward, codes, idents, isinstance(combine, tuple), why)
    empty = Program([], [], [], [], {})
    return PassPlan(field=None, monoid=codes[0], identity=idents[0], program=empty, generic=gp)


def _trace_pass(policy: Any, static: NetworkStatic, *, backward: bool) -> PassPlan:
    if isinstance(policy.combine, tuple):
        return _generic_pass(policy, backward=backward, why="a tuple accumulator")
    try:
        return _trace_product_pass(policy, static, backward=backward)
    except _NotProductForm as exc:
        return _generic_pass(policy, backward=backward, why=str(exc))


class _NotProductForm(UnsupportedPolicyError):
    """The map is outside the product form (the pass runs generic); other
    refusals -- an apply the tracer cannot follow -- stand."""


def _trace_product_pass(policy: Any, static: NetworkStatic, *, backward: bool) -> PassPlan:
    dtypes = _float_unit_fields(static)
    conn_dtypes = {s.name: np.dtype(s.dtype) for s in static.conn_fields}
    u = TraceUnitView(dtypes)
    c = TraceConnView(conn_dtypes)
    g = TraceGlobals(None)
    name = type(policy).__name__
    combine = policy.combine
    if not isinstance(combine, Monoid):
        raise UnsupportedPolicyError(f"{name}.combine must be a single named monoid")
    try:
        if backward:
            expr = policy.map(u, Index("src"), Index("dst"), c, Index("cid"), g)
            pm = product_map(expr, "dst")
        else:
            expr = policy.map(u, Index("dst"), Index("src"), c, Index("cid"), g)
            pm = product_map(expr, "src")
    except UnsupportedPolicyError as exc:
        raise _NotProductForm(str(exc)) from exc
    field = pm.field
    write = policy.apply(u, Index("self"), g, Expr("acc"))
    if not isinstance(write, UnitWrite):
        raise UnsupportedPolicyError(f"{name}.apply must return a UnitWrite")
    outs = list(write.fields.keys())
    prog = compile_program(list(write.fields.values()), outs, allow={"acc", "self"})
    _check_float_fields(outs + prog.fields + [field], dtypes, f"{name}")
    return PassPlan(field=field, monoid=combine.code, identity=combine.identity_for(), program=prog,
                    w_const=pm.w_const, x_const=pm.x_const)


def _trace_loss(loss: Any, static: NetworkStatic) -> LossPlan:
    dtypes = _float_unit_fields(static)
    seed_field = loss.seed_field.name
    _check_float_fields([seed_field], dtypes, type(loss).__name__)
    if isinstance(loss, SoftmaxCrossEntropyLoss):
        return LossPlan("softmax", seed_field)
    u = TraceUnitView(dtypes)
    out = loss.calculate_loss(u, Index("out"), Expr("target"), TraceGlobals(None))
    if not (isinstance(out, tuple) and len(out) == 2):
        raise UnsupportedPolicyError("calculate_loss must return (loss, seed)")
    value, seed = out
    if not (isinstance(value, Expr) and value.op == "sum"):
        raise UnsupportedPolicyError(
            "an elementwise loss must return jnp.sum(term) over the outputs as its value"
        )
    term = value.args[0]
    prog = compile_program([seed, term], [seed_field, None], allow={"target", "out", "fixed"})
    for k in prog.fixed_at.values():
        if k >= static.num_units:
            raise UnsupportedPolicyError(f"{type(loss).__name__} reads unit {k}; the net has {static.num_units}")
    _check_float_fields(prog.fields, dtypes, type(loss).__name__)
    return LossPlan("elementwise", seed_field, prog)


def compile_plan(net: type, static: NetworkStatic) -> Plan:
    """The device plan of ``net``'s streaming step."""
    for slot, method in (("update_unit", "update"), ("prune_unit", "predicate"), ("prune_conn", "predicate")):
        policy = getattr(net, slot, None)
        if policy is not None and not callable(getattr(policy, method, None)):
            raise TypeError(f"{net.__name__}.{slot} needs a {method} method")
    growth = GrowthConfig.of(net, static) if net.add_conn is not None else None
    if net.add_unit is not None:
        for name in ("spawn", "init"):
            if not callable(getattr(net.add_unit, name, None)):
                raise TypeError(f"{net.__name__}.add_unit needs a {name} method")
    if net.reset_global is not None and not callable(getattr(net.reset_global, "reset", None)):
        raise TypeError(f"{net.__name__}.reset_global needs a reset(g) method")
    forward = _trace_pass(net.forward_pass, static, backward=False)
    loss = _trace_loss(net.loss, static) if net.loss is not None else None
    backward = (
        _trace_pass(net.backward_pass, static, backward=True)
        if net.backward_pass is not None
        else None
    )
    update = None
    if net.update_conn is not None:
        uc = net.update_conn
        if not isinstance(uc, _RuleBase):
            for method in ("incoming", "outgoing"):
                if not callable(getattr(uc, method, None)):
                    raise TypeError(f"{net.__name__}.update_conn needs an {method} method")
            return Plan(forward, loss, backward, None, net=net, update_unit=net.update_unit is not None,
                        prune_unit=net.prune_unit is not None, prune_conn=net.prune_conn is not None,
                        add_unit=net.add_unit is not None, add_conn=growth,
                        reset_global=net.reset_global is not None, update_generic=True)
        dtypes = _float_unit_fields(static)
        _check_float_fields([uc.grad_field.name], dtypes, "update_conn")
        conn_names = {s.name for s in static.conn_fields}
        for col in uc.state_columns():
            if col not in conn_names:
                raise ValueError(
                    f"{net.__name__}: optimizer column {col!r} missing from extra_conn_fields"
                )
        update = uc
    return Plan(forward, loss, backward, update, net=net, update_unit=net.update_unit is not None,
                prune_unit=net.prune_unit is not None, prune_conn=net.prune_conn is not None,
                add_unit=net.add_unit is not None, add_conn=growth,
                reset_global=net.reset_global is not None)


def program_struct(
    prog: Program,
    units: dict,
    globals_: Any,
    *,
    out_override: dict | None = None,
    batch: int = 1,
    unit_map: np.ndarray | None = None,
) -> "_lib.plx_program":
    """The plx_program of ``prog`` over the given unit tensors (``batch`` > 1:
    columns of ``[num_units][batch]``; ``unit_map``: a fixed unit's logical
    id -> its row in renumbered columns)."""
    p = _lib.plx_program()
    p.ninstr = prog.ninstr
    p.nout = len(prog.out_fields)
    p.nfields = len(prog.fields)
    code = prog.flat_code()
    for k, v in enumerate(code):
        p.code[k] = int(v)
    for k, v in enumerate(prog.const_values(globals_)):
        p.consts[k] = float(v)
    mask = 0
    for k, name in enumerate(prog.fields):
        col = units[name]
        p.fields[k] = col.data_ptr()
        at = prog.fixed_at.get(k)
        if at is not None and unit_map is not None:
            at = int(unit_map[at])
        if at is not None:
            if (at + 1) * batch > col.numel():
                raise ValueError(f"unit {at} is outside the {name!r} column")
            p.fields[k] = col.data_ptr() + at * batch * col.element_size()
            mask |= 1 << k
    p.fixed_mask = mask
    over = out_override or {}
    for k, name in enumerate(prog.out_fields):
        if name is None:
            p.outs[k] = None
        else:
            p.outs[k] = (over[name] if name in over else units[name]).data_ptr()
    return p
