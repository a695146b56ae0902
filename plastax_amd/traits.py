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
from typing import Any, ClassVar, Generic, TypeVar

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


class ProposeAddConn:
    """Proposal-based connection growth (traits.py:576-682)."""


class ResetGlobal:
    """Global-state reset (traits.py:685-702)."""

    def reset(self, g: Any) -> Any:
        raise NotImplementedError


class BatchReduction:
    """How a batched step reduces per-sample unit columns (traits.py:705-871)."""


class MeanFloatFirstRest(BatchReduction):
    """Batch mean of floating columns, sample 0 of the rest."""


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
