"""Network state: the static jit key and the mutable struct of arrays.

Mirrors src/plastax/state.py:22-313. ``NetworkStatic`` is the hashable
configuration; ``NetworkState`` holds the unit columns, the connection
buckets and the scalar signals. Columns are torch tensors on the GPU
(``cuda:0``), or on the CPU for host-only construction.

Connection buckets are presented in the reference's *logical* slot order
(``state.conns[b][name]``) and unit columns in the caller's unit numbering.
The step itself runs on a physical, destination-sorted copy of the edges with
renumbered units (plastax_amd._layout.Arena): once a step has run, the unit
columns live in the arena's unit order and ``state.units`` is a read view in
the caller's numbering, rebuilt on first access after each step; the logical
connection columns are refreshed from the arena the same way.
"""

from __future__ import annotations

import dataclasses
from typing import Any

import numpy as np
import torch

from plastax_amd._types import PRUNED, FieldSpec, Propagation, ShardSpec

Columns = dict[str, torch.Tensor]


@dataclasses.dataclass(frozen=True)
class NetworkStatic:
    """Static network configuration (state.py:22-75)."""

    num_units: int
    propagation: Propagation
    unit_fields: tuple[FieldSpec, ...]
    conn_fields: tuple[FieldSpec, ...]
    level_capacities: tuple[int, ...]
    kahn_max_depth: int | None
    input_ids: tuple[int, ...]
    output_ids: tuple[int, ...]
    sharding: ShardSpec | None = None
    capacity_headroom: float = 0.0
    capacity_align: int | None = None
    seed: int = 0
    deepest_grows: bool = False


def torch_dtype(dtype: np.dtype) -> torch.dtype:
    """The torch dtype storing a column of numpy dtype ``dtype``."""
    dt = np.dtype(dtype)
    if dt == np.bool_:
        return torch.uint8
    return {
        np.dtype(np.float32): torch.float32,
        np.dtype(np.int32): torch.int32,
        np.dtype(np.uint32): torch.int32,
        np.dtype(np.float64): torch.float64,
        np.dtype(np.int64): torch.int64,
        np.dtype(np.uint8): torch.uint8,
    }[dt]


def default_device() -> torch.device:
    """``cuda:0`` when a GPU is visible, else the CPU."""
    return torch.device("cuda", 0) if torch.cuda.is_available() else torch.device("cpu")


def to_column(host: np.ndarray, spec: FieldSpec, device: torch.device) -> torch.Tensor:
    """Upload one host column with the storage dtype of ``spec``."""
    arr = np.ascontiguousarray(np.asarray(host).astype(spec.dtype, copy=False))
    if arr.dtype == np.bool_:
        arr = arr.view(np.uint8)
    elif arr.dtype == np.uint32:
        arr = arr.view(np.int32)
    return torch.from_numpy(arr.copy()).to(device)


def column_to_numpy(col: torch.Tensor, spec: FieldSpec) -> np.ndarray:
    """Download one column as a numpy array of the spec's dtype."""
    arr = col.detach().cpu().numpy()
    if np.dtype(spec.dtype) == np.bool_:
        return arr.astype(np.bool_)
    if np.dtype(spec.dtype) == np.uint32:
        return arr.view(np.uint32)
    return arr


_BOOL_FLAGS = frozenset({"needs_resort", "overflow", "unit_overflow"})


class NetworkState:
    """Mutable arena state (state.py:83-135).

    Attributes mirror the reference: ``units`` (name -> (num_units,) tensor),
    ``conns`` (one dict per bucket, logical slot order), ``globals_``,
    ``needs_resort``, ``step``, ``grown``, ``overflow``, ``units_added``,
    ``unit_overflow``, ``tail_start``. A state passed to a step is donated:
    the step reuses its buffers and the old object raises on access.
    """

    def __init__(
        self,
        units: Columns,
        conns: tuple[Columns, ...],
        globals_: Any,
        needs_resort: bool = False,
        step: int = 0,
        grown: int = 0,
        overflow: bool = False,
        units_added: int = 0,
        unit_overflow: bool = False,
        tail_start: int = 0,
    ) -> None:
        self._units = dict(units)
        self._conns: tuple[Columns, ...] = tuple(dict(b) for b in conns)
        self.globals_ = globals_
        self.step = step
        # The structural flags. A step leaves the ones its phases computed on
        # the device (_flag_dev: name -> (int32 device tensor, index)); the
        # first access reads that tensor once, so no step waits for them.
        self._flag_val: dict[str, Any] = {
            "needs_resort": needs_resort, "grown": grown, "overflow": overflow, "units_added": units_added,
            "unit_overflow": unit_overflow, "tail_start": tail_start}
        self._flag_dev: dict[str, tuple[Any, int]] = {}
        self._arena: Any = None  # plastax_amd._layout.Arena once a step ran
        self._arena_ahead = False  # the arena holds newer conn values
        # The churn layout a growth step replaced: the next layout is merged
        # from it (plastax_amd/_churn.py) instead of built from scratch.
        self._arena_prev: Any = None
        self._units_phys = False  # _units are in the arena's unit order
        self._units_view: Columns | None = None  # cached caller-order view
        self._donated = False

    # -- donation -------------------------------------------------------------
    def _check(self) -> None:
        if self._donated:
            raise RuntimeError(
                "this NetworkState was donated to a step; use the state in its StepResult"
            )

    def _donate(self) -> "NetworkState":
        """Hand every buffer to a fresh state object and retire this one."""
        self._check()
        new = NetworkState(self._units, self._conns, self.globals_, step=self.step)
        new._flag_val = dict(self._flag_val)
        new._flag_dev = dict(self._flag_dev)
        new._arena = self._arena
        new._arena_ahead = self._arena_ahead
        new._arena_prev = self._arena_prev
        new._units_phys = self._units_phys
        self._donated = True
        return new

    # -- structural flags ---------------------------------------------------------
    def _flag(self, name: str) -> Any:
        src = self._flag_dev.get(name)
        if src is not None:
            self._read_flags(src[0])
        return self._flag_val[name]

    def _set_flag(self, name: str, value: Any) -> None:
        """A host value (any pending device value of the flag is dropped)."""
        self._flag_dev.pop(name, None)
        self._flag_val[name] = value

    def _defer_flag(self, name: str, tensor: Any, index: int) -> None:
        """The flag is element ``index`` of the int32 device ``tensor``, read
        on first access."""
        self._flag_dev[name] = (tensor, int(index))

    def _flag_source(self, name: str) -> Any:
        """The flag's pending (device tensor, index), or None when its value
        is on the host."""
        return self._flag_dev.get(name)

    def _read_flags(self, tensor: Any) -> None:
        """One read of ``tensor`` resolves every flag pending on it. The
        caller waits on the device here anyway, so a churn arena's bounds
        are tightened to its counts at the same time (ChurnArena.reanchor)."""
        vals = tensor.cpu().tolist()
        for name, (t, i) in list(self._flag_dev.items()):
            if t is tensor:
                v = vals[i]
                self._flag_val[name] = bool(v) if name in _BOOL_FLAGS else int(v)
                del self._flag_dev[name]
        arena = self._arena_prev[0] if self._arena_prev else self._arena
        if hasattr(arena, "reanchor") and getattr(arena, "cols", None) is not None:
            arena.reanchor()

    def _flag_reader(self, name: str) -> Any:
        """A zero-argument callable giving the flag's value as of now, read
        from the device only when called (it holds no reference to the
        state, which a later step may donate)."""
        src = self._flag_dev.get(name)
        if src is None:
            value = self._flag_val[name]
            return lambda: value
        t, i = src
        kind = bool if name in _BOOL_FLAGS else int
        return lambda: kind(t[i].item())

    needs_resort = property(lambda self: self._flag("needs_resort"),
                            lambda self, v: self._set_flag("needs_resort", v))
    grown = property(lambda self: self._flag("grown"), lambda self, v: self._set_flag("grown", v))
    overflow = property(lambda self: self._flag("overflow"), lambda self, v: self._set_flag("overflow", v))
    units_added = property(lambda self: self._flag("units_added"), lambda self, v: self._set_flag("units_added", v))
    unit_overflow = property(lambda self: self._flag("unit_overflow"),
                             lambda self, v: self._set_flag("unit_overflow", v))
    tail_start = property(lambda self: self._flag("tail_start"), lambda self, v: self._set_flag("tail_start", v))

    def _mark_ahead(self, columns: Any = None) -> None:
        """The step wrote connection values into the arena: ``columns`` (a
        set of column names) or every column (None). The logical view is
        synchronised from the arena on its next access."""
        self._arena_ahead = True
        if self._arena is not None:
            self._arena.wrote(columns)

    def _physical_units(self, arena: Any) -> Columns:
        """The unit columns in ``arena``'s unit order (converted once); the
        step updates them in place, so the caller-order view is dropped."""
        if not self._units_phys:
            self._units = arena.units_to_physical(self._units)
            self._units_phys = True
        self._units_view = None
        return self._units

    # -- columns --------------------------------------------------------------
    @property
    def units(self) -> Columns:
        """Unit columns in the caller's unit numbering. After a step this is
        a read view of the device columns (rebuilt on first access after
        each step): assign ``state.units = {...}`` to change values."""
        self._check()
        if not self._units_phys:
            return self._units
        if self._units_view is None:
            self._units_view = self._arena.units_to_logical(self._units)
        return self._units_view

    @units.setter
    def units(self, value: Columns) -> None:
        self._check()
        self._units = dict(value)
        self._units_phys = False
        self._units_view = None

    @property
    def conns(self) -> tuple[Columns, ...]:
        """Connection buckets in logical slot order (synchronised from the
        device arena on first access after a step)."""
        self._check()
        if self._arena is not None and self._arena_ahead:
            self._arena.write_logical(self._conns)
            self._arena_ahead = False
        return self._conns

    @conns.setter
    def conns(self, value: tuple[Columns, ...]) -> None:
        self._check()
        if self._units_phys:  # the next arena may number units differently
            self._units = self.units
            self._units_phys = False
            self._units_view = None
        self._conns = tuple(dict(b) for b in value)
        self._arena = None  # structure or values changed on the host side
        self._arena_ahead = False
        self._arena_prev = None

    @property
    def device(self) -> torch.device:
        return next(iter(self._units.values())).device

    def __repr__(self) -> str:
        if self._donated:
            return "NetworkState(<donated>)"
        caps = tuple(int(next(iter(b.values())).shape[0]) for b in self._conns)
        return f"NetworkState(units={len(self._units)} cols, buckets={caps}, step={self.step})"


def _filled(specs: tuple[FieldSpec, ...], n: int, device: torch.device) -> Columns:
    return {s.name: to_column(np.full((n,), s.default, dtype=s.dtype), s, device) for s in specs}


def make_empty_state(static: NetworkStatic, globals_: Any, device: Any = None) -> NetworkState:
    """Arenas at capacity with every connection slot dead (state.py:148-177)."""
    dev = torch.device(device) if device is not None else default_device()
    units = _filled(static.unit_fields, static.num_units, dev)
    conns = tuple(_filled(static.conn_fields, c, dev) for c in static.level_capacities)
    return NetworkState(units, conns, globals_)


def live_conn_count(state: NetworkState, level: int | None = None) -> int:
    """Live connections in one bucket or all (state.py:180-198)."""
    buckets = state.conns if level is None else (state.conns[level],)
    return int(sum(int((b["dead"] == 0).sum()) for b in buckets))


def live_unit_mask(units: Columns) -> torch.Tensor | None:
    """Unit slots holding a live unit, or None without a unit capacity
    (state.py:201-219)."""
    pruned = units.get(PRUNED.name)
    return None if pruned is None else pruned == 0


def live_unit_count(state: NetworkState) -> int:
    """Live units (state.py:222-235)."""
    live = live_unit_mask(state.units)
    if live is None:
        return int(next(iter(state.units.values())).shape[0])
    return int(live.sum())


def grow_bucket(static: NetworkStatic, state: NetworkState, level: int) -> tuple[NetworkStatic, NetworkState]:
    """Pad one bucket with never-used (DEAD, default) slots (state.py:238-313).

    The new capacity is ``max(capacity_policy(live + 1), floor)`` with the
    floor twice the old capacity (1.5x, aligned, under ``capacity_align``),
    so repeated overflows cost O(log) regrows. In PIPELINE mode the padding
    extends the never-used tail; ``tail_start`` stays. The state's buffers
    are handed to the returned state (the old one is retired).
    """
    import dataclasses as _dc

    from plastax_amd.topo import capacity_policy

    conns = state.conns  # logical columns, synchronised from the device arena
    old = int(static.level_capacities[level])
    live = int((conns[level]["dead"] == 0).sum())
    policy = capacity_policy(live + 1, headroom=static.capacity_headroom, align=static.capacity_align)
    if static.capacity_align is None:
        floor = old * 2
    else:
        floor = capacity_policy(old + old // 2, align=static.capacity_align)
    new_cap = max(policy, floor)
    pad = new_cap - old
    specs = {s.name: s for s in static.conn_fields}
    grown = {}
    for name, col in conns[level].items():
        fill = to_column(np.full((pad,), specs[name].default, dtype=specs[name].dtype), specs[name], col.device)
        grown[name] = torch.cat([col, fill])
    new_conns = tuple(grown if b == level else dict(c) for b, c in enumerate(conns))
    caps = tuple(new_cap if b == level else c for b, c in enumerate(static.level_capacities))
    new_static = _dc.replace(static, level_capacities=caps)
    units = state.units
    new_state = NetworkState(
        dict(units), new_conns, state.globals_, state.needs_resort, state.step, state.grown,
        state.overflow, state.units_added, state.unit_overflow, state.tail_start,
    )
    state._donated = True
    return new_static, new_state
