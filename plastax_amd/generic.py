"""Passes outside the product form (sweep.py:113-230, :343-449 with any map
and combine).

The fast kernels take a map of the product form ``(WEIGHT or a constant) *
(a unit field at the other end or a constant)`` and one named monoid. Any
other pass -- a nonlinear map (``w * f(x[src])``), a map reading other
connection columns, a tuple accumulator with a tuple of monoids (the
reference's examples xmc.py, upgd.py, cbp.py) -- runs here:

- the map is traced into an edge program with one float32 output per
  accumulator component (``_site.trace_pass_map``);
- ``plx_gen_fold`` folds each row's entries in order, one thread per row:
  a forward row is a destination, its entries the slab range of its
  in-edges (slot order); a backward row a source, its entries its out-edges
  in slot order (the churn layout's lists, or on a tiled arena the
  per-source lists of ``batched.batch_sources``); each component from its
  monoid's identity, then combined into the carried accumulator columns;
- the apply is traced into a unit program reading the accumulator from
  those columns (``_site.trace_pass_apply``), evaluated for the units the
  bucket finalizes against the pre-apply columns, its writes committed with
  ``plx_unit_write`` (pruned units skipped), and the finalized units'
  accumulators reset to the identity.

The finalize sets are the product path's: forward, level b + 1 after bucket
b (PIPELINE: every non-input unit after one sweep); backward, the deepest
level from the identity, then level b after bucket b down to 1 (PIPELINE:
every unit after one sweep).

Under a batched step (``batch`` B > 1) every unit column the programs read
and the accumulators are ``[num_units][B]``: the fold runs one thread per
(row, sample), the apply one site per (finalized unit, sample), and each
sample's writes land at ``unit * B + sample`` (step.py:443-447 runs the
pass per sample against the shared connections).
"""

from __future__ import annotations

import ctypes
from typing import Any

import numpy as np
import torch

from plastax_amd import _lib, _site
from plastax_amd._expr import UnsupportedPolicyError
from plastax_amd._plan import GenericPass


class GenericPassRunner:
    """A traced generic pass, bound to a net's columns."""

    def __init__(self, gp: GenericPass, static: Any, globals_: Any) -> None:
        self.gp = gp
        self.static = static
        self.k = len(gp.monoids)
        unit_dtypes = {s.name: np.dtype(s.dtype) for s in static.unit_fields}
        conn_dtypes = {s.name: np.dtype(s.dtype) for s in static.conn_fields}
        name = type(gp.policy).__name__
        self.map_prog = _site.trace_pass_map(gp.policy, gp.backward, unit_dtypes, conn_dtypes, globals_)
        if len(self.map_prog.out_kinds) != self.k:
            raise UnsupportedPolicyError(
                f"{name}.map returns {len(self.map_prog.out_kinds)} components; combine has {self.k}")
        self.apply_prog, self.names = _site.trace_pass_apply(gp.policy, self.k, gp.tuple_acc, unit_dtypes,
                                                             globals_)
        self.acc_names = _site.acc_field_names(self.k)
        self.specs = {s.name: s for s in static.unit_fields}

    def new_acc(self, n: int, device: torch.device, batch: int = 1) -> list[torch.Tensor]:
        return [torch.full((n * batch,), v, dtype=torch.float32, device=device) for v in self.gp.identities]

    def check_columns(self, units: dict, batch: int) -> None:
        """Every unit column the programs read holds ``num_units * batch``
        entries (the kernels index ``unit * batch + sample``)."""
        want = self.static.num_units * batch
        for name in list(self.map_prog.unit_fields) + list(self.apply_prog.unit_fields):
            if name in self.acc_names:
                continue
            col = units.get(name)
            if col is None or col.numel() != want:
                have = None if col is None else col.numel()
                raise ValueError(f"generic pass: unit column {name!r} holds {have} entries, the pass reads {want}")

    def fold(self, k: Any, arena: Any, b: int, units: dict, acc: list[torch.Tensor], g: Any, *,
             rows: torch.Tensor, nrows: int, ptr: torch.Tensor, entry_pos: torch.Tensor | None,
             batch: int = 1) -> None:
        """One bucket's rows folded into ``acc`` (per sample when batched)."""
        from plastax_amd.grow import fill_prog

        if nrows == 0:
            return
        base, cap = arena.bases[b], arena.caps[b]
        view = {name: col[base : base + cap] for name, col in arena.cols.items()}
        d = _lib.plx_gen_fold_desc()
        d.prog = fill_prog(self.map_prog, units, view, g, physical_ids=True)
        d.nrows, d.ncomp, d.backward = int(nrows), self.k, int(self.gp.backward)
        d.batch = int(batch)
        d.num_units = self.static.num_units
        for j in range(self.k):
            d.monoid[j] = self.gp.monoids[j]
            d.identity[j] = self.gp.identities[j]
            d.acc[j] = acc[j].data_ptr()
        d.row_unit, d.row_ptr = rows.data_ptr(), ptr.data_ptr()
        d.entry_pos = None if entry_pos is None else entry_pos.data_ptr()
        d.from_id, d.to_id = arena.cols["from_id"].data_ptr(), arena.cols["to_id"].data_ptr()
        # (list entries may name tombstoned positions; tiled rows hold them
        # only when the arena says so)
        d.dead = arena.cols["dead"].data_ptr() if arena.dead_in_rows or entry_pos is not None else None
        d.base = base
        d.slot = arena.slot[base:].data_ptr()
        d.ids_logical, d.ids_physical = arena.uperm32.data_ptr(), arena.uinv32.data_ptr()
        _lib.check(k.lib.plx_gen_fold(d, k.s), "plx_gen_fold")

    def apply(self, k: Any, arena: Any, units: dict, acc: list[torch.Tensor], g: Any,
              fin: torch.Tensor, batch: int = 1, pruned: torch.Tensor | None = None) -> None:
        """The apply on the units ``fin`` (physical ids), against the
        pre-apply columns; their accumulators go back to the identity.
        Pruned units (``pruned``, else the ``pruned`` column) keep their
        columns."""
        from plastax_amd.grow import _ptr
        from plastax_amd.units import _unit_cols

        m = int(fin.numel())
        if m == 0:
            return
        B = int(batch)
        if pruned is None:
            pruned = units.get("pruned")
        ext = dict(units)
        ext.update(dict(zip(self.acc_names, acc)))
        idx = fin.long()
        if self.names:
            n = m * B
            at, skip = fin, pruned
            if B > 1:  # sites (unit, sample), written at unit * B + sample
                at = (idx[:, None] * B + torch.arange(B, device=idx.device)).reshape(-1).to(torch.int32)
                skip = None if pruned is None else pruned.repeat_interleave(B)
            outs = [k.mem.i32(n) for _ in self.names]
            k.site_eval(self.apply_prog, ext, g, n=n, kind=0, per=1, num_units=self.static.num_units, outs=outs,
                        site_ids=arena.uperm32[idx].contiguous(), ids_physical=arena.uinv32, batch=B)
            cols = _unit_cols(units, self.specs, self.names)
            ptrs = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
            _lib.check(k.lib.plx_unit_write(n, None, at.data_ptr(), _ptr(skip), len(self.names),
                                            ctypes.addressof(cols), ctypes.addressof(ptrs), k.s), "plx_unit_write")
        for a, v in zip(acc, self.gp.identities):
            a.view(-1, B).index_fill_(0, idx, v)


def finalize_lists(arena: Any, static: Any) -> dict[str, list[torch.Tensor]]:
    """Per arena: the units each bucket's apply finalizes (physical ids),
    forward and backward (see the module docstring)."""
    cache = arena.__dict__.get("_generic_fin")
    if cache is not None:
        return cache
    levels = arena.unit_levels
    n = levels.size
    is_input = np.zeros(n, dtype=bool)
    if static.input_ids:
        is_input[arena.uinv[np.asarray(static.input_ids, dtype=np.int64)]] = True
    nb = arena.num_buckets

    def lst(mask: np.ndarray) -> torch.Tensor:
        return torch.from_numpy(np.flatnonzero(mask).astype(np.int32)).to(arena.device)

    if arena.pipeline:
        fwd = [lst(~is_input)]
        bwd = [lst(np.ones(n, dtype=bool))]
    else:
        fwd = [lst((levels == b + 1) & ~is_input) for b in range(nb)]
        bwd = [lst((levels == b) & ~is_input) for b in range(nb + 1)]  # bwd[nb]: the deepest level
    cache = {"fwd": fwd, "bwd": bwd}
    arena._generic_fin = cache
    return cache
