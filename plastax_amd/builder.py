"""Host-side network construction (src/plastax/builder.py:80-661).

``NetworkBuilder.from_edges`` buckets edges by source level, orders each
bucket source-major (stable argsort of ``src * N + dst``, builder.py:566-579)
and pads it with tombstones to ``capacity_policy`` (topo.py:455-506): the
reference's logical arena, byte for byte. The device copies the columns to
the GPU; the step builds its destination-sorted physical copy from them.
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from typing import Any

import numpy as np

from plastax_amd import topo
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
from plastax_amd.state import NetworkState, NetworkStatic, default_device, to_column


class NetworkBuilder:
    """Construct a network host-side (builder.py:80-128)."""

    def __init__(self, net: type, globals_: Any) -> None:
        self.net = net
        self.globals_ = globals_
        self._unit_fields: tuple[FieldSpec, ...] = (
            ACTIVATION,
            LEVEL,
            *((PRUNED,) if net.unit_capacity is not None else ()),
            *net.extra_unit_fields,
        )
        self._conn_fields: tuple[FieldSpec, ...] = (
            FROM_ID,
            TO_ID,
            DEAD,
            WEIGHT,
            *net.extra_conn_fields,
        )
        self._settable_unit_fields = {
            s.name: s for s in self._unit_fields if s.name not in (LEVEL.name, PRUNED.name)
        }
        self._settable_conn_fields = {
            s.name: s
            for s in self._conn_fields
            if s.name not in (FROM_ID.name, TO_ID.name, DEAD.name)
        }
        self._units: list[dict[str, Any]] = []
        self._conn_src: list[int] = []
        self._conn_dst: list[int] = []
        self._conn_values: list[dict[str, Any]] = []
        self._input_ids: list[int] = []
        self._output_ids: list[int] = []

    @classmethod
    def from_edges(
        cls,
        net: type,
        num_units: int,
        from_ids: np.ndarray,
        to_ids: np.ndarray,
        *,
        weights: np.ndarray | None = None,
        input_ids: Sequence[int],
        output_ids: Sequence[int],
        globals_: Any,
        extra_conn_columns: Mapping[str, np.ndarray] | None = None,
        capacity_headroom: float = 0.0,
        capacity_align: int | None = None,
        sharding: ShardSpec | None = None,
        device: Any = None,
    ) -> tuple[NetworkStatic, NetworkState]:
        """Build arenas from whole edge-column arrays (builder.py:177-300)."""
        builder = cls(net, globals_)
        src_arr = np.asarray(from_ids, dtype=np.int32)
        dst_arr = np.asarray(to_ids, dtype=np.int32)
        if src_arr.ndim != 1 or dst_arr.shape != src_arr.shape:
            raise ValueError(
                "from_edges: from_ids and to_ids must be 1-D arrays of equal "
                f"length, got {src_arr.shape} and {dst_arr.shape}"
            )
        num_edges = int(src_arr.shape[0])
        extra = dict(extra_conn_columns or {})
        for name in extra:
            if name not in builder._settable_conn_fields or name == WEIGHT.name:
                raise ValueError(
                    f"from_edges: unknown or non-settable conn field {name!r} in extra_conn_columns"
                )
        conn_columns: dict[str, np.ndarray] = {}
        for name, spec in builder._settable_conn_fields.items():
            supplied = np.asarray(weights) if (name == WEIGHT.name and weights is not None) else extra.get(name)
            if supplied is None:
                conn_columns[name] = np.full((num_edges,), spec.default, dtype=spec.dtype)
            elif np.asarray(supplied).shape != (num_edges,):
                raise ValueError(
                    f"from_edges: conn column {name!r} has shape {np.asarray(supplied).shape}, "
                    f"expected ({num_edges},)"
                )
            else:
                conn_columns[name] = np.asarray(supplied)
        unit_columns = {
            name: np.full((num_units,), spec.default, dtype=spec.dtype)
            for name, spec in builder._settable_unit_fields.items()
        }
        return builder._assemble(
            num_units,
            src_arr,
            dst_arr,
            conn_columns,
            unit_columns,
            tuple(int(i) for i in input_ids),
            tuple(int(i) for i in output_ids),
            capacity_headroom=capacity_headroom,
            capacity_align=capacity_align,
            sharding=sharding,
            device=device,
        )

    def add_unit(self, **field_values: Any) -> int:
        """Add a unit, unset fields at their defaults (builder.py:302-325)."""
        for name in field_values:
            if name not in self._settable_unit_fields:
                raise ValueError(f"add_unit: unknown or non-settable unit field {name!r}")
        self._units.append(
            {n: field_values.get(n, s.default) for n, s in self._settable_unit_fields.items()}
        )
        return len(self._units) - 1

    def add_conn(self, src: int, dst: int, **field_values: Any) -> None:
        """Add a connection (builder.py:327-348)."""
        for name in field_values:
            if name not in self._settable_conn_fields:
                raise ValueError(f"add_conn: unknown or non-settable conn field {name!r}")
        self._conn_src.append(int(src))
        self._conn_dst.append(int(dst))
        self._conn_values.append(
            {n: field_values.get(n, s.default) for n, s in self._settable_conn_fields.items()}
        )

    def mark_input(self, unit_id: int) -> None:
        self._input_ids.append(int(unit_id))

    def mark_output(self, unit_id: int) -> None:
        self._output_ids.append(int(unit_id))

    def finalize(
        self,
        *,
        capacity_headroom: float = 0.0,
        capacity_align: int | None = None,
        sharding: ShardSpec | None = None,
        device: Any = None,
    ) -> tuple[NetworkStatic, NetworkState]:
        """Freeze the accumulated units and connections (builder.py:358-414)."""
        num_units = len(self._units)
        src_arr = np.asarray(self._conn_src, dtype=np.int32)
        dst_arr = np.asarray(self._conn_dst, dtype=np.int32)
        conn_columns = {
            n: np.asarray([row[n] for row in self._conn_values], dtype=s.dtype)
            for n, s in self._settable_conn_fields.items()
        }
        unit_columns = {
            n: np.asarray([row[n] for row in self._units], dtype=s.dtype)
            for n, s in self._settable_unit_fields.items()
        }
        return self._assemble(
            num_units,
            src_arr,
            dst_arr,
            conn_columns,
            unit_columns,
            tuple(self._input_ids),
            tuple(self._output_ids),
            capacity_headroom=capacity_headroom,
            capacity_align=capacity_align,
            sharding=sharding,
            device=device,
        )

    def _assemble(
        self,
        num_units: int,
        src_arr: np.ndarray,
        dst_arr: np.ndarray,
        conn_columns: dict[str, np.ndarray],
        unit_columns: dict[str, np.ndarray],
        input_ids: tuple[int, ...],
        output_ids: tuple[int, ...],
        *,
        capacity_headroom: float = 0.0,
        capacity_align: int | None = None,
        sharding: ShardSpec | None = None,
        device: Any = None,
    ) -> tuple[NetworkStatic, NetworkState]:
        """Bucket, sort and pad the edge columns (builder.py:416-661)."""
        if sharding is not None or self.net.sharding is not None:
            raise NotImplementedError("Scheme-A sharding: this build runs on one GPU")
        dev = default_device() if device is None else device
        capacity = self.net.unit_capacity
        num_slots = num_units if capacity is None else capacity
        if num_slots < num_units:
            raise ValueError(
                f"finalize: {self.net.__name__}.unit_capacity {capacity} is below the "
                f"{num_units} built units"
            )
        for unit_id in (*input_ids, *output_ids):
            if not 0 <= unit_id < num_units:
                raise ValueError(f"finalize: unit id {unit_id} out of range [0, {num_units})")
        if src_arr.size:
            lo = min(int(src_arr.min()), int(dst_arr.min()))
            hi = max(int(src_arr.max()), int(dst_arr.max()))
            if lo < 0 or hi >= num_units:
                raise ValueError(f"finalize: an edge endpoint is out of range [0, {num_units})")
        edges = np.stack([src_arr, dst_arr], axis=1) if src_arr.size else np.zeros((0, 2), np.int32)
        pipeline = self.net.propagation is Propagation.PIPELINE
        levels = topo.initial_levels(
            num_units, edges, allow_cycles=pipeline, input_ids=tuple(input_ids)
        )

        unit_cols = {}
        for spec in self._unit_fields:
            if spec.name == PRUNED.name:
                host = np.arange(num_slots) >= num_units
            else:
                vals = levels if spec.name == LEVEL.name else unit_columns[spec.name]
                host = np.asarray(vals, dtype=spec.dtype)
                if num_slots > num_units:
                    host = np.concatenate(
                        [host, np.full((num_slots - num_units,), spec.default, spec.dtype)]
                    )
            unit_cols[spec.name] = to_column(host, spec, dev)

        if pipeline:
            bucket_of_conn = np.zeros_like(src_arr)
            num_buckets = 1
            deepest_grows = False
        else:
            bucket_of_conn = levels[src_arr] if src_arr.size else src_arr
            max_level = int(levels.max()) if levels.size else 0
            deepest_grows = self.net.add_conn is not None
            num_buckets = max(max_level + (1 if deepest_grows else 0), 1)

        conns = []
        level_capacities = []
        live_total = 0
        for level_idx in range(num_buckets):
            idx = np.flatnonzero(bucket_of_conn == level_idx)
            # Source-major order, ties by destination, stable for parallel
            # edges (builder.py:566-579).
            key = src_arr[idx].astype(np.int64) * num_units + dst_arr[idx]
            order = idx[np.argsort(key, kind="stable")]
            live = int(order.size)
            live_total += live
            cap = topo.capacity_policy(live, headroom=capacity_headroom, align=capacity_align)
            cols = {}
            for spec in self._conn_fields:
                if spec.name == FROM_ID.name:
                    vals = src_arr[order]
                elif spec.name == TO_ID.name:
                    vals = dst_arr[order]
                elif spec.name == DEAD.name:
                    vals = np.zeros((live,), dtype=np.bool_)
                else:
                    vals = np.asarray(conn_columns[spec.name])[order]
                host = np.concatenate(
                    [
                        np.asarray(vals).astype(spec.dtype),
                        np.full((cap - live,), spec.default, dtype=spec.dtype),
                    ]
                )
                cols[spec.name] = to_column(host, spec, dev)
            conns.append(cols)
            level_capacities.append(cap)

        static = NetworkStatic(
            num_units=num_slots,
            propagation=self.net.propagation,
            unit_fields=self._unit_fields,
            conn_fields=self._conn_fields,
            level_capacities=tuple(level_capacities),
            kahn_max_depth=self.net.kahn_max_depth,
            input_ids=input_ids,
            output_ids=output_ids,
            sharding=None,
            capacity_headroom=capacity_headroom,
            capacity_align=capacity_align,
            seed=self.net.seed,
            deepest_grows=deepest_grows,
        )
        state = NetworkState(
            unit_cols,
            tuple(conns),
            self.globals_,
            tail_start=live_total if pipeline else 0,
        )
        return static, state
