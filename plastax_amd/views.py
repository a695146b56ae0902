"""Read views and write records of a policy call (src/plastax/views.py:25-120).

Policies receive a ``UnitView`` ``u`` and a ``ConnView`` ``c`` and read
``u[FIELD, unit]`` / ``c[FIELD, cid]``; they return ``UnitWrite.of(...)`` or
``ConnWrite.of(...)``. While a step is being built the views are the symbolic
ones of plastax_amd._expr, so the same policy code is traced once and runs on
the device.
"""

from __future__ import annotations

import dataclasses
from typing import Any

from plastax_amd._expr import TraceConnView as ConnView  # noqa: F401
from plastax_amd._expr import TraceUnitView as UnitView  # noqa: F401
from plastax_amd._types import FieldSpec


@dataclasses.dataclass(frozen=True)
class UnitWrite:
    """The unit columns an apply writes (views.py:80-99)."""

    fields: dict[str, Any]

    @staticmethod
    def of(*pairs: tuple[FieldSpec, Any]) -> "UnitWrite":
        return UnitWrite({spec.name: value for spec, value in pairs})


@dataclasses.dataclass(frozen=True)
class ConnWrite:
    """The connection columns an update writes (views.py:102-120)."""

    fields: dict[str, Any]

    @staticmethod
    def of(*pairs: tuple[FieldSpec, Any]) -> "ConnWrite":
        return ConnWrite({spec.name: value for spec, value in pairs})
