"""Named monoids (src/plastax/monoid.py:22-218).

A forward or backward pass declares how its per-edge values combine per
unit. The device folds them with the named op; ``sum_``, ``prod``, ``max_``
and ``min_`` carry the same identities as the reference (0, 1, -inf, +inf).
A generic ``Monoid(op, identity)`` has no lowering, as in the reference.
"""

from __future__ import annotations

import dataclasses
import enum
import math
from typing import Any, Callable


class UnsupportedMonoidError(NotImplementedError):
    """A monoid the device cannot lower (monoid.py:217)."""


class _Named(enum.Enum):
    SUM = "sum"
    PROD = "prod"
    MAX = "max"
    MIN = "min"


_IDENTITY = {
    _Named.SUM: 0.0,
    _Named.PROD: 1.0,
    _Named.MAX: -math.inf,
    _Named.MIN: math.inf,
}
# Device code of each named monoid (PLX_MONOID_* in include/plastax_hip.h).
_CODE = {_Named.SUM: 0, _Named.PROD: 1, _Named.MAX: 2, _Named.MIN: 3}


@dataclasses.dataclass(frozen=True)
class Monoid:
    """Associative combine with identity (monoid.py:63-214)."""

    named: _Named | None
    op: Callable[[Any, Any], Any] | None = None
    identity: Any = None

    @property
    def code(self) -> int:
        """The device code of this monoid."""
        if self.named is None:
            raise UnsupportedMonoidError(
                "generic Monoid(op, identity) has no lowering; only named "
                "monoids (sum/prod/max/min) are supported"
            )
        return _CODE[self.named]

    def identity_for(self, dtype: Any = None) -> float:
        """The identity element (as a Python float)."""
        if self.named is None:
            raise UnsupportedMonoidError("generic Monoid has no identity lowering")
        return _IDENTITY[self.named]


sum_ = Monoid(_Named.SUM)
prod = Monoid(_Named.PROD)
max_ = Monoid(_Named.MAX)
min_ = Monoid(_Named.MIN)

__all__ = ["Monoid", "UnsupportedMonoidError", "max_", "min_", "prod", "sum_"]
