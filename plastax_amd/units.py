"""The unit phases on the device: update_unit, prune_unit, add_unit.

Host orchestration of the unit-lifecycle entry points of csrc/structural.hip,
mirroring the reference's phases (phases.py:1148-1193 update_unit,
:1245-1307 prune_unit, :1310-1441 add_unit). The policies are traced into
site programs (plastax_amd._site) and evaluated once per unit slot.

update_unit and prune_unit work on the step's unit columns in whatever order
they are stored: given the arena's renumbering, the program sees the
caller's ids (``site_ids``, ``ids_physical``) while reading and writing each
unit at its own position. add_unit ranks parents and free slots by id, so it
works on the caller's numbering (logical unit columns).
"""

from __future__ import annotations

import ctypes
from typing import Any

import numpy as np
import torch

from plastax_amd import _lib, _site
from plastax_amd.grow import Kernels, _ptr

Columns = dict[str, torch.Tensor]


def _unit_cols(units: Columns, specs: dict, names: list[str]) -> Any:
    cols = (_lib.plx_unit_col * max(1, len(names)))()
    for k, name in enumerate(names):
        col = units[name]
        cols[k].ptr = col.data_ptr()
        cols[k].bytes = 1 if col.element_size() == 1 else 4
        v = np.asarray(specs[name].default).astype(specs[name].dtype)
        cols[k].default_bits = int(bool(v)) if v.dtype == np.bool_ else int(v.view(np.uint32))
    return cols


def _reset_names(static: Any) -> list[str]:
    """Unit columns a pruned or new slot resets to its default (LEVEL and
    PRUNED are set by the phase itself)."""
    names = []
    for s in static.unit_fields:
        if s.name in ("level", "pruned"):
            continue
        if np.dtype(s.dtype).itemsize not in (1, 4):
            raise TypeError(f"unit column {s.name!r}: only 32-bit and bool columns are supported")
        names.append(s.name)
    if len(names) > _lib.PLX_MAX_UNIT_COLS:
        raise ValueError(f"at most {_lib.PLX_MAX_UNIT_COLS} resettable unit columns")
    return names


class UpdateUnitPhase:
    """Every live unit's update against the pre-phase columns."""

    def __init__(self, net: Any, static: Any, globals_: Any) -> None:
        self.static = static
        self.specs = {s.name: s for s in static.unit_fields}
        dtypes = {s.name: np.dtype(s.dtype) for s in static.unit_fields}
        self.prog, self.names = _site.trace_update_unit(net.update_unit, dtypes, globals_)

    def run(self, k: Kernels, units: Columns, globals_: Any, *, site_ids: torch.Tensor | None = None,
            ids_physical: torch.Tensor | None = None, batch: int = 1, skip: torch.Tensor | None = None) -> None:
        """With batch > 1 the unit columns are a batched step's [num_units][B]
        per-sample columns (every sample updated against its own values) and
        ``skip`` is the matching [num_units][B] PRUNED mask."""
        n_units = int(units["level"].shape[0]) if batch == 1 else int(next(iter(units.values())).shape[0])
        n = n_units * batch
        if not self.names:
            return
        outs = [k.mem.i32(n) for _ in self.names]
        k.site_eval(self.prog, units, globals_, n=n, kind=0, per=1, num_units=n_units, outs=outs,
                    site_ids=site_ids, ids_physical=ids_physical, batch=batch)
        cols = _unit_cols(units, self.specs, self.names)
        ptrs = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
        mask = units.get("pruned") if batch == 1 else skip
        _lib.check(k.lib.plx_unit_write(n, None, None, _ptr(mask), len(self.names),
                                        ctypes.addressof(cols), ctypes.addressof(ptrs), k.s), "plx_unit_write")


class PruneUnitPhase:
    """Prune the selected live units that are neither inputs nor outputs."""

    def __init__(self, net: Any, static: Any, globals_: Any) -> None:
        self.static = static
        self.specs = {s.name: s for s in static.unit_fields}
        dtypes = {s.name: np.dtype(s.dtype) for s in static.unit_fields}
        self.prog = _site.trace_prune_unit(net.prune_unit, dtypes, globals_)
        self.names = _reset_names(static)
        n = static.num_units
        m = np.zeros(n, np.uint8)
        m[np.asarray(tuple(static.input_ids) + tuple(static.output_ids), dtype=np.int64)] = 1
        self._exempt_host = m

    def exempt(self, device: torch.device, order: torch.Tensor | None) -> torch.Tensor:
        """The input/output mask, in the caller's order or through ``order``
        (physical position -> caller's id); the last one is kept while the
        same ``order`` tensor comes back (an arena's numbering)."""
        last = self.__dict__.get("_exempt_last")
        if last is not None and last[0] == device and last[1] is order:
            return last[2]
        t = torch.from_numpy(self._exempt_host).to(device)
        t = t if order is None else t[order.long()].contiguous()
        self._exempt_last = (device, order, t)
        return t

    def run(self, k: Kernels, units: Columns, globals_: Any, *, site_ids: torch.Tensor | None = None,
            ids_physical: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Marks the doomed units; returns (doomed mask, doomed count), both
        on the device, in the columns' own order."""
        n = int(units["level"].shape[0])
        selected = k.mem.i32(n)
        k.site_eval(self.prog, units, globals_, n=n, kind=0, per=1, num_units=n, outs=[selected],
                    site_ids=site_ids, ids_physical=ids_physical)
        doomed = k.mem.u8(n)
        count = torch.zeros(1, dtype=torch.int32, device=selected.device)
        cols = _unit_cols(units, self.specs, self.names)
        ex = self.exempt(selected.device, site_ids)
        _lib.check(k.lib.plx_unit_prune(n, selected.data_ptr(), units["pruned"].data_ptr(), ex.data_ptr(),
                                        len(self.names), ctypes.addressof(cols), doomed.data_ptr(), count.data_ptr(),
                                        k.s), "plx_unit_prune")
        return doomed, count

    @staticmethod
    def kill_columns(k: Kernels, n: int, from_id: torch.Tensor, to_id: torch.Tensor, dead: torch.Tensor,
                     doomed: torch.Tensor, kills: torch.Tensor | None = None) -> None:
        """The incident-edge kill over n slots of one bucket's columns (unit
        ids in the numbering of ``doomed``)."""
        _lib.check(k.lib.plx_kill_incident(n, from_id.data_ptr(), to_id.data_ptr(), dead.data_ptr(),
                                           doomed.data_ptr(), None, None if kills is None else kills.data_ptr(),
                                           None, 0.0, k.s), "plx_kill_incident")

    @staticmethod
    def kill(k: Kernels, arena: Any, doomed: torch.Tensor, kills: torch.Tensor | None = None) -> None:
        """The incident-edge kill on the physical arena, bucket by bucket
        (physical unit ids on both sides); an edge killed in a bucket whose
        Adam step count is kept as one number gets that number in its own
        column (arena.stamp_target)."""
        cols = arena.cols
        for b in range(arena.num_buckets):
            # Positions past the live range are dead slots: nothing to kill there.
            base, span = arena.bases[b], arena.lives[b]
            if span == 0:
                continue
            stamp, value = arena.stamp_target(b)
            _lib.check(k.lib.plx_kill_incident(span, cols["from_id"][base:].data_ptr(), cols["to_id"][base:].data_ptr(),
                                               cols["dead"][base:].data_ptr(), doomed.data_ptr(), None,
                                               None if kills is None else kills.data_ptr(),
                                               None if stamp is None else stamp.data_ptr(), float(value), k.s),
                       "plx_kill_incident")


class AddUnitPhase:
    """Children of the spawning live units, placed in the lowest free slots."""

    def __init__(self, net: Any, static: Any, globals_: Any) -> None:
        self.static = static
        self.specs = {s.name: s for s in static.unit_fields}
        dtypes = {s.name: np.dtype(s.dtype) for s in static.unit_fields}
        self.spawn = _site.trace_spawn(net.add_unit, dtypes, globals_)
        self.init, self.init_names = _site.trace_unit_init(net.add_unit, dtypes, globals_)
        self.names = _reset_names(static)
        self.max_level = int(getattr(net, "max_levels", 1024)) - 1
        self.interval = int(getattr(net, "structural_interval", 1))
        # the level offset a spawn gives its children, when the policy
        # returns a traced constant (None: computed per parent)
        self.offset_const = self.spawn.const_output(1)

    def level_bound(self, bound: int) -> int:
        """A bound on the deepest level after this phase, given one before:
        a child's level is clamp(parent + offset, 1, max_level)."""
        c = self.offset_const
        child = self.max_level if c is None else min(self.max_level, max(bound + c, 1))
        return max(bound, child)

    def fires(self, step: int) -> bool:
        return self.interval <= 1 or step % self.interval == 0

    def run(self, k: Kernels, units: Columns, globals_: Any) -> tuple[int, bool]:
        """On the caller's unit numbering; returns (units_added,
        unit_overflow) (a host read)."""
        got = self.run_device(k, units, globals_).cpu().tolist()
        return int(got[0]), bool(got[1])

    def run_device(self, k: Kernels, units: Columns, globals_: Any) -> torch.Tensor:
        """run() without the host read: returns the device flags
        (units_added, unit_overflow) as two int32."""
        n = int(units["level"].shape[0])
        wants, offset = k.mem.i32(n), k.mem.i32(n)
        k.site_eval(self.spawn, units, globals_, n=n, kind=0, per=1, num_units=n, outs=[wants, offset])
        parents, nparents = k.compact(n, 3, wants)  # PLX_FLAG_I32
        free, nfree = k.compact(n, 0, units["pruned"])  # PLX_FLAG_U8: the slots free before the phase
        child, parent = k.mem.i32(n), k.mem.i32(n)
        flags = torch.zeros(2, dtype=torch.int32, device=wants.device)
        cols = _unit_cols(units, self.specs, self.names)
        _lib.check(k.lib.plx_unit_place(n, parents.data_ptr(), nparents.data_ptr(), free.data_ptr(), nfree.data_ptr(),
                                        offset.data_ptr(), units["level"].data_ptr(), units["pruned"].data_ptr(),
                                        self.max_level, len(self.names), ctypes.addressof(cols), child.data_ptr(),
                                        parent.data_ptr(), flags.data_ptr(), k.s), "plx_unit_place")
        if self.init_names:
            outs = [k.mem.i32(n) for _ in self.init_names]
            k.site_eval(self.init, units, globals_, n=n, kind=4, num_units=n, list_a=child, list_b=parent,
                        n_dev=flags, outs=outs)
            icols = _unit_cols(units, self.specs, self.init_names)
            ptrs = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
            _lib.check(k.lib.plx_unit_write(n, flags.data_ptr(), child.data_ptr(), None, len(self.init_names),
                                            ctypes.addressof(icols), ctypes.addressof(ptrs), k.s), "plx_unit_write")
        return flags

