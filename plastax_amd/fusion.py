"""Prune-into-forward fusion (phases.py:1517-1541, :1629-1848, :2322-2469).

``plan_prune_fusion`` decides, from the traced policies, whether
``prune_conn.predicate`` may be evaluated inside the forward sweep, where it
sees the state before loss, backward, update_unit and update_conn ran. That
is legal when

- the predicate's reads (its unit and connection fields, and DEAD, which the
  prune merges into) are not written by any phase between the forward and
  the prune: the loss (its seed column), the backward's apply, update_unit,
  update_conn;
- every unit field it reads that the forward's apply writes is "forwarded":
  its post-forward value depends only on the unit id, the globals and unit
  columns the forward does not write (not on the accumulator), so it is
  computed before the sweep from the identity accumulator;
- no prune_unit runs (its tombstones come before prune_conn).

Execution (both commit the tombstones at the prune slot, so loss, backward
and update still see the old DEAD; ``plx_merge_kills``):

- ``"hip"``: one edge pass per bucket. The forward kernel evaluates the
  predicate for every position it folds and leaves it in a sink column
  (``plx_forward_desc.prune_prog``), reading DEAD once for both; the
  predicate is compiled into the kernel (``plx_forward_prune_compile``,
  hipRTC) or, if that fails, interpreted by ``plx_forward_bucket``.
  ``fuse_prune="auto"`` and ``"triton"`` take it (it stands in for the
  reference's single-pass Triton kernel).
- ``"xla"``: the predicate pass runs at the forward's slot as a separate
  edge pass (the reference's portable lowering, which reads the edge columns
  twice).

A fused step's state is bit-identical to the two-pass step's.
"""

from __future__ import annotations

import dataclasses
from typing import Any

import numpy as np

from plastax_amd._expr import Expr, Index, TraceGlobals, TraceUnitView
from plastax_amd._types import DEAD, WEIGHT
from plastax_amd.views import UnitWrite

ENGINES = ("auto", "triton", "xla", "hip")


@dataclasses.dataclass(frozen=True)
class PruneFusionPlan:
    """Whether and how prune_conn runs inside the forward sweep
    (phases.py:1517-1541): ``engine`` "hip" or "xla" when fused;
    ``forwarded`` the unit fields computed before the sweep."""

    fused: bool
    reason: str
    engine: str | None = None
    forwarded: tuple[str, ...] = ()


@dataclasses.dataclass
class PruneFusionRecord:
    """What a step decided (``StepFn.prune_fusion``; planned on its first
    call, against the globals)."""

    requested: str
    plan: PruneFusionPlan | None = None


def _leaves(e: Any, out: set[tuple[str, str | None]]) -> set[tuple[str, str | None]]:
    """The leaves of a traced expression: ("acc", None), ("ldu", field), ..."""
    if isinstance(e, Expr):
        if e.op in ("acc", "ldu", "global", "target"):
            out.add((e.op, e.field))
        for a in e.args:
            _leaves(a, out)
    return out


def _apply_writes(policy: Any, unit_dtypes: dict) -> dict[str, Any]:
    """A pass's apply(u, i, g, acc) as {written field: traced value}."""
    write = policy.apply(TraceUnitView(unit_dtypes), Index("self"), TraceGlobals(None), Expr("acc"))
    if not isinstance(write, UnitWrite):
        raise TypeError(f"{type(policy).__name__}.apply must return a UnitWrite")
    return dict(write.fields)


def plan_prune_fusion(net: type, static: Any, globals_: Any, *, engine: str = "auto") -> PruneFusionPlan:
    """Decide, from the traced policies, whether prune_conn can run inside
    the forward sweep (phases.py:1629-1848). ``engine``: "triton" / "hip"
    (the single-pass kernel: the forward evaluates the predicate at every
    position it folds), "xla" (the predicate as its own pass at the
    forward's slot, its kills staged in a sink and merged at the prune
    slot), or "auto": not fused -- on this device the predicate pass at the
    prune slot, the predicate compiled to its own kernel (four sites per
    lane, ORing straight into DEAD), is the fastest (C2 with a PruneConn
    every step: 1.03 ms per step, against 1.38 for "triton", whose forward
    kernel has the predicate compiled in and takes 77 us per bucket where
    the forward alone takes 29 and the separate pass 16, and a sink to
    merge for "xla"); the results are the same bits every way."""
    if engine not in ENGINES:
        raise ValueError(f"plan_prune_fusion: unknown engine {engine!r}")
    from plastax_amd import _site
    from plastax_amd.optim._rules import _RuleBase

    pc = net.prune_conn
    if pc is None:
        return PruneFusionPlan(False, "no prune_conn")
    if net.prune_unit is not None:
        return PruneFusionPlan(False, "prune_unit tombstones edges before prune_conn")
    unit_dtypes = {s.name: np.dtype(s.dtype) for s in static.unit_fields}
    conn_dtypes = {s.name: np.dtype(s.dtype) for s in static.conn_fields}
    try:
        pred = _site.trace_predicate(pc, unit_dtypes, conn_dtypes, globals_)
        reads = {("unit", n) for n in pred.unit_fields} | {("conn", n) for n in pred.conn_fields}
        reads.add(("conn", DEAD.name))
        fwd = _apply_writes(net.forward_pass, unit_dtypes)
        between: set[tuple[str, str]] = set()
        if net.loss is not None:
            between.add(("unit", net.loss.seed_field.name))
        if net.backward_pass is not None:
            between |= {("unit", k) for k in _apply_writes(net.backward_pass, unit_dtypes)}
        if net.update_unit is not None:
            _, names = _site.trace_update_unit(net.update_unit, unit_dtypes, globals_)
            between |= {("unit", k) for k in names}
        uc = net.update_conn
        if uc is not None:
            if isinstance(uc, _RuleBase):
                between |= {("conn", WEIGHT.name)} | {("conn", k) for k in uc.state_columns()}
            else:
                for d in ("incoming", "outgoing"):
                    _, names = _site.trace_conn_update(getattr(uc, d), d, unit_dtypes, static.conn_fields,
                                                       globals_)
                    between |= {("conn", k) for k in names}
        clash = sorted(name for _, name in reads & between)
        if clash:
            return PruneFusionPlan(False, f"a phase between forward and prune writes {clash}")
        forwarded = tuple(sorted(name for kind, name in reads if kind == "unit" and name in fwd))
        for name in forwarded:
            for op, field in sorted(_leaves(fwd[name], set()), key=str):
                if op == "acc":
                    return PruneFusionPlan(
                        False, f"predicate reads {name!r}, which the forward computes from its accumulator")
                if op == "ldu" and field in fwd:
                    return PruneFusionPlan(
                        False, f"predicate reads {name!r}, which the forward computes from {field!r}, "
                        "itself written by the forward")
    except Exception as exc:  # noqa: BLE001 - a policy that does not trace is not provably safe
        return PruneFusionPlan(False, f"could not trace the policies: {exc!r}")
    if engine == "xla":
        return PruneFusionPlan(True, "legal; the predicate pass at the forward's slot (requested)", "xla", forwarded)
    if engine == "auto":
        return PruneFusionPlan(False, "legal, not fused: the predicate pass at the prune slot is the fastest "
                               "engine on this device")
    return PruneFusionPlan(True, "legal; one edge pass (HIP forward)", "hip", forwarded)
