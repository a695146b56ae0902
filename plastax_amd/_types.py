"""Core shared types: column specs, built-in columns, propagation modes.

Mirrors the reference's ``_types.py`` (src/plastax/_types.py:30-132): a
network is a struct of arrays, one column per :class:`FieldSpec`, over the
units and over each connection bucket. Index types are plain ints here; the
device columns are torch tensors on the GPU.
"""

from __future__ import annotations

import dataclasses
import enum
from typing import Any, NewType

import numpy as np

UnitIdx = NewType("UnitIdx", int)
ConnIdx = NewType("ConnIdx", int)
Level = NewType("Level", int)


class Propagation(enum.Enum):
    """Sweep scheduling mode (_types.py:39-43)."""

    TOPOLOGICAL = "topological"
    PIPELINE = "pipeline"


@dataclasses.dataclass(frozen=True)
class ShardSpec:
    """Scheme-A sharding config (_types.py:46-62). Accepted for signature
    compatibility; this build runs one GPU and rejects a non-None spec."""

    axis_name: str
    num_shards: int


@dataclasses.dataclass(frozen=True)
class FieldSpec:
    """One SoA column: name, numpy dtype and the fill value of fresh rows
    (_types.py:65-115)."""

    name: str
    dtype: np.dtype
    default: Any

    @staticmethod
    def field(name: str, dtype: Any, default: Any) -> "FieldSpec":
        """A column spec for an arbitrary numpy scalar dtype."""
        dt = np.dtype(dtype)
        return FieldSpec(name, dt, dt.type(default))

    @staticmethod
    def float32(name: str, default: float = 0.0) -> "FieldSpec":
        """A float32 column spec."""
        return FieldSpec.field(name, np.float32, default)

    @staticmethod
    def int32(name: str, default: int = 0) -> "FieldSpec":
        """An int32 column spec."""
        return FieldSpec.field(name, np.int32, default)

    @staticmethod
    def boolean(name: str, default: bool = False) -> "FieldSpec":
        """A boolean column spec."""
        return FieldSpec.field(name, np.bool_, default)


# Built-in connection columns (_types.py:118-122).
FROM_ID = FieldSpec.int32("from_id")
TO_ID = FieldSpec.int32("to_id")
DEAD = FieldSpec.boolean("dead", default=True)
WEIGHT = FieldSpec.float32("weight")

# Built-in unit columns (_types.py:125-132).
ACTIVATION = FieldSpec.float32("activation")
LEVEL = FieldSpec.int32("level")
PRUNED = FieldSpec.boolean("pruned", default=True)
