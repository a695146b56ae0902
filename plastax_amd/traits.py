"""The declarative surface: policy protocols and the Network base class.

Mirrors src/plastax/traits.py. A network is a ``Network`` subclass whose
class attributes name its policies (traits.py:874-949); absent slots are
elided. The policies' callbacks are traced when a step is built (see
plastax_amd._expr): forward/backward maps must be the linear
``WEIGHT * field[other]`` form, applies and elementwise losses compile to
device programs, and connection updates must be one of the optim bundles.
"""

from __future__ import annotations

import dataclasses
import enum
from collections.abc import Mapping
from typing import Any, ClassVar, Generic, NamedTuple, TypeVar

import numpy as np

from plastax_amd import monoid as _monoid
from plastax_amd._expr import UnsupportedPolicyError
from plastax_amd._types import (
    ACTIVATION,
    DEAD,
    FROM_ID,
    LEVEL,
    PRUNED,
    TO_ID,
    WEIGHT,
    FieldSpec,
    Propagation,
    ShardSpec,
)

GS = TypeVar("GS")


class ForwardPass:
    """Forward propagation policy (traits.py:38-88): ``combine`` monoid,
    ``map(u, dst, src, c, cid, g)`` per edge, ``apply(u, i, g, acc)`` per unit."""

    combine: Any = _monoid.sum_
    linear_input: FieldSpec | None = None

    def map(self, u: Any, dst: Any, src: Any, c: Any, cid: Any, g: Any) -> Any:
        raise NotImplementedError

    def apply(self, u: Any, i: Any, g: Any, acc: Any) -> Any:
        raise NotImplementedError


class BackwardPass:
    """Backward propagation policy (traits.py:91-150): ``map(u, src, dst, c,
    cid, g)`` accumulates into the source; ``apply`` runs per unit."""

    combine: Any = _monoid.sum_
    linear_input: FieldSpec | None = None

    def map(self, u: Any, src: Any, dst: Any, c: Any, cid: Any, g: Any) -> Any:
        raise NotImplementedError

    def apply(self, u: Any, i: Any, g: Any, acc: Any) -> Any:
        raise NotImplementedError


class Loss:
    """Loss policy (traits.py:153-201): ``calculate_loss(u, outputs, targets,
    g) -> (loss, seed)``; the seed lands in ``seed_field`` at the outputs."""

    seed_field: FieldSpec

    def calculate_loss(self, u: Any, outputs: Any, targets: Any, g: Any) -> Any:
        raise NotImplementedError


@dataclasses.dataclass(frozen=True)
class SoftmaxCrossEntropyLoss:
    """Softmax over the outputs, cross-entropy against the targets
    (traits.py:204-250): seed = exp(z)/s - t, loss = sum(t * (log s - z))."""

    seed_field: FieldSpec


class UpdateUnit:
    """Per-unit update after backward (traits.py:253-278)."""

    def update(self, u: Any, i: Any, g: Any) -> Any:
        raise NotImplementedError


class UpdateConn:
    """Per-edge update (traits.py:281-348): ``incoming`` then ``outgoing``."""

    def incoming(self, u: Any, dst: Any, src: Any, c: Any, cid: Any, g: Any) -> Any:
        raise NotImplementedError

    def outgoing(self, u: Any, src: Any, dst: Any, c: Any, cid: Any, g: Any) -> Any:
        raise NotImplementedError


class PruneConn:
    """Connection pruning predicate (traits.py:351-373)."""

    def predicate(self, u: Any, c: Any, cid: Any, g: Any) -> Any:
        raise NotImplementedError


class PruneUnit:
    """Unit pruning predicate (traits.py:376-405)."""

    def predicate(self, u: Any, i: Any, g: Any) -> Any:
        raise NotImplementedError


class AddUnit:
    """Unit addition policy (traits.py:408-463)."""


class ScoreAddConn:
    """Scored connection growth (traits.py:466-551)."""


class Proposal(NamedTuple):
    """One growth proposal (traits.py:554-566): a directed candidate edge and
    its priority. ``propose`` may return one (or a plain ``(src, dst,
    score)`` tuple); a ``-inf`` score vetoes the candidate."""

    src: Any
    dst: Any
    score: Any


class ProposeAddConn:
    """Proposal-based connection growth (traits.py:576-682)."""


class ResetGlobal:
    """Global-state reset (traits.py:685-702)."""

    def reset(self, g: Any) -> Any:
        raise NotImplementedError


class Reduction(enum.Enum):
    """How a batched step combines one unit column's per-sample values
    (traits.py:705-720): MEAN (the sum over the samples in order, then divided
    by B; floating columns only), SUM (numeric, non-boolean), FIRST (sample
    0), NOT_BATCHED (no per-sample phase may write the column; it keeps its
    pre-step value)."""

    MEAN = "mean"
    SUM = "sum"
    FIRST = "first"
    NOT_BATCHED = "not_batched"


class BatchReduction:
    """A batch-reduction policy (traits.py:723-754): ``reduction(field)``
    returns the column's Reduction, or None when it is undeclared. Any object
    with a callable ``reduction`` satisfies it."""

    def reduction(self, field: FieldSpec) -> "Reduction | None":
        raise NotImplementedError

    @classmethod
    def __subclasshook__(cls, other: type) -> bool:
        return callable(getattr(other, "reduction", None))


class FieldReductions(BatchReduction):
    """Declares unit columns one by one (traits.py:755-808)."""

    def __init__(self, fields: Mapping[FieldSpec, Reduction]) -> None:
        pairs = tuple(fields.items())
        names: set[str] = set()
        for spec, red in pairs:
            if not isinstance(spec, FieldSpec):
                raise TypeError(f"FieldReductions: {spec!r} is not a FieldSpec")
            if not isinstance(red, Reduction):
                raise TypeError(f"FieldReductions: {spec.name!r} maps to {red!r}, not a Reduction")
            if spec.name in names:
                raise ValueError(f"FieldReductions: {spec.name!r} declared twice")
            names.add(spec.name)
        self.fields = pairs

    def reduction(self, field: FieldSpec) -> "Reduction | None":
        for spec, red in self.fields:
            if spec.name == field.name:
                return red
        return None


class MeanFloatFirstRest(BatchReduction):
    """MEAN for every floating unit column, FIRST for the others, NOT_BATCHED
    for LEVEL and PRUNED (traits.py:811-834)."""

    def reduction(self, field: FieldSpec) -> Reduction:
        if field.name in _STRUCTURAL_UNIT_FIELDS:
            return Reduction.NOT_BATCHED
        if np.issubdtype(np.dtype(field.dtype), np.floating):
            return Reduction.MEAN
        return Reduction.FIRST


# Unit columns only the structural phases write: never reduced over a batch.
_STRUCTURAL_UNIT_FIELDS = frozenset({"level", "pruned"})


def batch_written_reduction(policy: Any, field: FieldSpec, *, where: str) -> Reduction:
    """The reduction of a column a per-sample phase writes, or ValueError
    (traits.py:841-871)."""
    red = policy.reduction(field)
    if red is None:
        raise ValueError(
            f"batch_reduction: unit column {field.name!r} is written per sample ({where}) but the "
            "batch-reduction policy does not declare it; declare it MEAN, SUM or FIRST (or set "
            "batch_reduction = MeanFloatFirstRest())")
    if red is Reduction.NOT_BATCHED:
        raise ValueError(
            f"batch_reduction: unit column {field.name!r} is declared NOT_BATCHED but is written "
            f"per sample ({where})")
    return red


_RESERVED = frozenset(
    {FROM_ID.name, TO_ID.name, DEAD.name, WEIGHT.name, ACTIVATION.name, LEVEL.name, PRUNED.name}
)


class Network(Generic[GS]):
    """Base configuration surface for a network's traits (traits.py:874-949)."""

    forward_pass: ClassVar[Any]
    backward_pass: ClassVar[Any] = None
    loss: ClassVar[Any] = None
    update_unit: ClassVar[Any] = None
    update_conn: ClassVar[Any] = None
    prune_unit: ClassVar[Any] = None
    prune_conn: ClassVar[Any] = None
    add_unit: ClassVar[Any] = None
    add_conn: ClassVar[Any] = None
    reset_global: ClassVar[Any] = None

    extra_unit_fields: ClassVar[tuple[FieldSpec, ...]] = ()
    extra_conn_fields: ClassVar[tuple[FieldSpec, ...]] = ()
    propagation: ClassVar[Propagation] = Propagation.TOPOLOGICAL
    kahn_max_depth: ClassVar[int | None] = None
    sharding: ClassVar[ShardSpec | None] = None
    seed: ClassVar[int] = 0
    structural_interval: ClassVar[int] = 1
    unit_capacity: ClassVar[int | None] = None
    max_levels: ClassVar[int] = 1024
    batch_reduction: ClassVar[BatchReduction | None] = None

    def __init_subclass__(cls, **kwargs: Any) -> None:
        super().__init_subclass__(**kwargs)
        _validate_traits(cls)


def _validate_traits(cls: type) -> None:
    """Field-name checks of _validate_traits (traits.py:1072-1160)."""
    seen: set[str] = set()
    for spec in (*cls.extra_unit_fields,):
        if spec.name in _RESERVED:
            raise ValueError(f"{cls.__name__}: unit field name {spec.name!r} is reserved")
        if spec.name in seen:
            raise ValueError(f"{cls.__name__}: duplicate unit field {spec.name!r}")
        seen.add(spec.name)
    seen = set()
    for spec in (*cls.extra_conn_fields,):
        if spec.name in _RESERVED:
            raise ValueError(f"{cls.__name__}: conn field name {spec.name!r} is reserved")
        if spec.name in seen:
            raise ValueError(f"{cls.__name__}: duplicate conn field {spec.name!r}")
        seen.add(spec.name)
    if cls.structural_interval < 1:
        raise ValueError(f"{cls.__name__}.structural_interval must be >= 1")
    if cls.sharding is not None:
        raise UnsupportedPolicyError("Scheme-A sharding: this build runs on one GPU")
    for name in ("prune_unit", "add_unit"):
        if getattr(cls, name) is not None and cls.unit_capacity is None:
            raise ValueError(f"{cls.__name__}.{name} requires unit_capacity")
    if cls.unit_capacity is not None and cls.unit_capacity < 1:
        raise ValueError(f"{cls.__name__}.unit_capacity must be positive")
    for spec in (*cls.extra_unit_fields, *cls.extra_conn_fields):
        if not isinstance(spec, FieldSpec):
            raise TypeError(f"{cls.__name__}: extra fields must be FieldSpec, got {spec!r}")
        np.dtype(spec.dtype)
    _validate_batch_reduction(cls)


def _validate_batch_reduction(cls: type) -> None:
    """The policy against the network's unit columns (traits.py:1177-1248)."""
    policy = getattr(cls, "batch_reduction", None)
    if policy is None:
        return
    if not callable(getattr(policy, "reduction", None)) or isinstance(policy, type):
        raise TypeError(f"{cls.__name__}.batch_reduction must satisfy BatchReduction (reduction); got {policy!r}")
    unit_fields = (ACTIVATION, LEVEL, *((PRUNED,) if cls.unit_capacity is not None else ()),
                   *cls.extra_unit_fields)
    if isinstance(policy, FieldReductions):
        known = {spec.name for spec in unit_fields}
        for spec, _ in policy.fields:
            if spec.name not in known:
                raise ValueError(f"{cls.__name__}.batch_reduction declares {spec.name!r}, which is not a unit "
                                 f"column of the network ({sorted(known)})")
    for spec in unit_fields:
        red = policy.reduction(spec)
        if red is None or red is Reduction.NOT_BATCHED:
            continue
        if not isinstance(red, Reduction):
            raise TypeError(f"{cls.__name__}.batch_reduction.reduction({spec.name!r}) must return a Reduction "
                            f"or None; got {red!r}")
        if spec.name in _STRUCTURAL_UNIT_FIELDS:
            raise ValueError(f"{cls.__name__}.batch_reduction: {spec.name!r} is written only by the structural "
                             f"phases; declare it NOT_BATCHED or leave it undeclared, not {red.name}")
        dt = np.dtype(spec.dtype)
        if red is Reduction.MEAN and not np.issubdtype(dt, np.floating):
            raise TypeError(f"{cls.__name__}.batch_reduction: MEAN needs a floating column; {spec.name!r} is {dt}")
        if red is Reduction.SUM and (dt == np.bool_ or not np.issubdtype(dt, np.number)):
            raise TypeError(f"{cls.__name__}.batch_reduction: SUM needs a numeric, non-boolean column; "
                            f"{spec.name!r} is {dt}")
    try:
        batch_written_reduction(policy, ACTIVATION, where="the input scatter")
        if cls.loss is not None:
            batch_written_reduction(policy, cls.loss.seed_field, where="the loss's seed_field")
    except ValueError as err:
        raise ValueError(f"{cls.__name__}.{err}") from None
