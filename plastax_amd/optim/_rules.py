"""SGD, Momentum, Adam(W) and RMSProp bundles.

Each ``_*UpdateConn`` holds the rule's float32 constants and names its state
columns; the device applies the rule in one fused pass (``plx_update_conn``)
with the reference's float32 operation order:

- SGD: ``w - lr * g`` (optim/_sgd.py:121-126)
- Momentum: ``v = mu * v + g; w - lr * v`` (optim/_momentum.py:136-139)
- Adam(W): optim/_adam.py:154-172, with ``b ** t`` a float32 power of the
  float32 step column
- RMSProp: ``s = d * s + (1 - d) * g * g; w - lr * g / sqrt(s + eps)``
  (optim/_rmsprop.py:135-140)

The gradient of every rule is ``grad_field[dst] * activation[src]``.
"""

from __future__ import annotations

import dataclasses
from typing import Any, Protocol, runtime_checkable

import numpy as np

from plastax_amd._types import FieldSpec
from plastax_amd.views import ConnWrite

_f32 = np.float32

# Per-connection optimizer state columns (all default 0.0).
OPT_M = FieldSpec.float32("opt/m")
OPT_V = FieldSpec.float32("opt/v")
OPT_T = FieldSpec.float32("opt/t")


@runtime_checkable
class Optimizer(Protocol):
    """An UpdateConn policy plus the state columns it needs
    (optim/__init__.py:47-77)."""

    state_fields: tuple[FieldSpec, ...]
    needs_step_counter: bool

    def update_conn(self) -> Any: ...


class _RuleBase:
    """The device rule code and the incoming/outgoing protocol surface."""

    rule_code: int = -1
    grad_field: FieldSpec

    def incoming(self, u: Any, dst: Any, src: Any, c: Any, cid: Any, g: Any) -> ConnWrite:
        raise NotImplementedError("optim rules run fused on the device")

    def outgoing(self, u: Any, src: Any, dst: Any, c: Any, cid: Any, g: Any) -> ConnWrite:
        return ConnWrite.of()

    def state_columns(self) -> tuple[str, ...]:
        return ()


@dataclasses.dataclass(frozen=True)
class _SGDUpdateConn(_RuleBase):
    lr: float
    grad_field: FieldSpec
    rule_code = 0

    def params(self) -> list[np.float32]:
        return [_f32(self.lr)]


@dataclasses.dataclass(frozen=True)
class _MomentumUpdateConn(_RuleBase):
    lr: float
    momentum: float
    grad_field: FieldSpec
    velocity: FieldSpec = OPT_V
    rule_code = 1

    def params(self) -> list[np.float32]:
        return [_f32(self.lr), _f32(self.momentum)]

    def state_columns(self) -> tuple[str, ...]:
        return (self.velocity.name,)


@dataclasses.dataclass(frozen=True)
class _AdamUpdateConn(_RuleBase):
    lr: float
    b1: float
    b2: float
    eps: float
    weight_decay: float
    grad_field: FieldSpec
    m: FieldSpec = OPT_M
    v: FieldSpec = OPT_V
    t: FieldSpec = OPT_T
    rule_code = 2

    def params(self) -> list[np.float32]:
        # jnp.float32(1.0 - self.b1): the difference is taken in float64 and
        # rounded once (_adam.py:163-164).
        return [
            _f32(self.lr),
            _f32(self.b1),
            _f32(self.b2),
            _f32(self.eps),
            _f32(self.weight_decay),
            _f32(1.0 - self.b1),
            _f32(1.0 - self.b2),
        ]

    def state_columns(self) -> tuple[str, ...]:
        return (self.m.name, self.v.name, self.t.name)


@dataclasses.dataclass(frozen=True)
class _RMSPropUpdateConn(_RuleBase):
    lr: float
    decay: float
    eps: float
    grad_field: FieldSpec
    mean_sq: FieldSpec = OPT_V
    rule_code = 3

    def params(self) -> list[np.float32]:
        return [_f32(self.lr), _f32(self.decay), _f32(1.0 - self.decay), _f32(self.eps)]

    def state_columns(self) -> tuple[str, ...]:
        return (self.mean_sq.name,)


@dataclasses.dataclass(frozen=True)
class SGD:
    """Stateless SGD bundle (optim/_sgd.py:152-199)."""

    lr: float
    grad_field: FieldSpec
    state_fields: tuple[FieldSpec, ...] = ()
    needs_step_counter: bool = False

    def update_conn(self) -> _SGDUpdateConn:
        return _SGDUpdateConn(self.lr, self.grad_field)


@dataclasses.dataclass(frozen=True)
class Momentum:
    """Heavy-ball momentum bundle (optim/_momentum.py:160-212)."""

    lr: float
    momentum: float
    grad_field: FieldSpec
    state_fields: tuple[FieldSpec, ...] = (OPT_V,)
    needs_step_counter: bool = False

    def update_conn(self) -> _MomentumUpdateConn:
        return _MomentumUpdateConn(self.lr, self.momentum, self.grad_field)


@dataclasses.dataclass(frozen=True)
class Adam:
    """Adam(W) bundle with per-connection moments and step (optim/_adam.py:196-248)."""

    lr: float
    grad_field: FieldSpec
    b1: float = 0.9
    b2: float = 0.999
    eps: float = 1e-8
    weight_decay: float = 0.0
    state_fields: tuple[FieldSpec, ...] = (OPT_M, OPT_V, OPT_T)
    needs_step_counter: bool = False

    def update_conn(self) -> _AdamUpdateConn:
        return _AdamUpdateConn(
            self.lr, self.b1, self.b2, self.eps, self.weight_decay, self.grad_field
        )


@dataclasses.dataclass(frozen=True)
class RMSProp:
    """Uncentered RMSProp bundle (optim/_rmsprop.py:160-223)."""

    lr: float
    grad_field: FieldSpec
    decay: float = 0.9
    eps: float = 1e-8
    state_fields: tuple[FieldSpec, ...] = (OPT_V,)
    needs_step_counter: bool = False

    def update_conn(self) -> _RMSPropUpdateConn:
        return _RMSPropUpdateConn(self.lr, self.decay, self.eps, self.grad_field)


def sgd(lr: float, grad_field: FieldSpec) -> SGD:
    """A stateless SGD optimizer (optim/_sgd.py:185-199)."""
    return SGD(lr=lr, grad_field=grad_field)


def momentum(lr: float, momentum: float, grad_field: FieldSpec) -> Momentum:
    """A heavy-ball momentum optimizer (optim/_momentum.py:196-212)."""
    return Momentum(lr=lr, momentum=momentum, grad_field=grad_field)


def adam(
    lr: float, grad_field: FieldSpec, *, b1: float = 0.9, b2: float = 0.999, eps: float = 1e-8
) -> Adam:
    """An Adam optimizer (optim/_adam.py:251-273)."""
    return Adam(lr=lr, grad_field=grad_field, b1=b1, b2=b2, eps=eps)


def adamw(
    lr: float,
    grad_field: FieldSpec,
    *,
    weight_decay: float = 1e-4,
    b1: float = 0.9,
    b2: float = 0.999,
    eps: float = 1e-8,
) -> Adam:
    """An AdamW optimizer: Adam with decoupled weight decay (optim/_adam.py:276-298)."""
    return Adam(lr=lr, grad_field=grad_field, b1=b1, b2=b2, eps=eps, weight_decay=weight_decay)


def rmsprop(
    lr: float, grad_field: FieldSpec, *, decay: float = 0.9, eps: float = 1e-8
) -> RMSProp:
    """An RMSProp optimizer (optim/_rmsprop.py:203-223)."""
    return RMSProp(lr=lr, grad_field=grad_field, decay=decay, eps=eps)
