"""The churn layout: a physical arena rebuilt on the device after every
structural change.

A net whose growth fires every step (C5's reservoir) changes its arena every
step, and the tiled layout's host build (unit renumbering, tiles, groups,
hot / cold partials) would dominate the step. The churn layout keeps what the
forward and the update need and replaces the backward's tiles with
slot-ordered lists, so the whole build is a few ordered compactions, two
stable radix sorts and gathers, all on the device:

- units keep the caller's ids (no renumbering; the gathers get no LDS table);
- positions ``[base_b, base_b + live_b)`` hold bucket b's live edges sorted by
  (destination, slot), then its dead slots in slot order (the tiled layout's
  slab, so the forward and the update kernels are unchanged);
- every unit is a forward row (offsets by an integer histogram and scan of
  the destinations); rows that neither receive nor finalize pass their
  accumulator through unchanged;
- the backward walks each source's live out-edges in logical slot order --
  the reference's own scatter order (sweep.py:343-399) -- from copies of
  TO_ID (fixed by the build) and of WEIGHT / liveness (gathered each step
  before the update).
"""

from __future__ import annotations

import numpy as np
import torch

from plastax_amd import _lib
from plastax_amd._layout import PAD, Arena, ForwardRows, _round_up
from plastax_amd._types import DEAD, FROM_ID, TO_ID, Propagation
from plastax_amd.state import Columns, NetworkStatic, torch_dtype


class SourceLists:
    """Bucket b's backward lists: row r (unit r) owns entries
    ``[ptr[r], ptr[r+1])``, entry j being physical position ``pos[j]`` with
    TO_ID ``dst[j]``; ``weight`` / ``live`` are refreshed each step."""

    def __init__(self, ptr: torch.Tensor, pos: torch.Tensor, dst: torch.Tensor) -> None:
        self.ptr = ptr
        self.pos = pos
        self.dst = dst
        n = int(pos.numel())
        self.weight = torch.empty(n, dtype=torch.float32, device=pos.device)
        self.live = torch.empty(n, dtype=torch.uint8, device=pos.device)


class ChurnArena(Arena):
    """A physical arena built on the device from the logical buckets."""

    churn = True

    def __init__(self, static: NetworkStatic, units: Columns, conns: tuple[Columns, ...],
                 device: torch.device, stream: int) -> None:
        from plastax_amd.grow import Kernels

        self.static = static
        self.device = device
        self.tile = 0
        self.nsuper = 0
        n = static.num_units
        nb = len(conns)
        self.num_buckets = nb
        self.pipeline = static.propagation is Propagation.PIPELINE
        k = Kernels(device, stream)
        ident = np.arange(n, dtype=np.int64)
        self.uperm = ident
        self.uinv = ident
        self.uperm_t = torch.arange(n, dtype=torch.int64, device=device)
        self.uinv_t = self.uperm_t
        self.uperm32 = self.uperm_t.to(torch.int32)
        self.uinv32 = self.uperm32
        levels = units["level"]
        self.unit_levels = levels.cpu().numpy().astype(np.int64)
        self.lvl_start = np.zeros(1, np.int64)
        self.input_ids = self._i32(np.asarray(static.input_ids, dtype=np.int64))
        self.output_ids = self._i32(np.asarray(static.output_ids, dtype=np.int64))
        is_input = np.zeros(n, dtype=np.uint8)
        if static.input_ids:
            is_input[np.asarray(static.input_ids)] = 1
        self.is_input = torch.from_numpy(is_input).to(device)
        caps = [int(b[DEAD.name].numel()) for b in conns]
        spans = [_round_up(c, 4) for c in caps]
        bases = np.concatenate([[0], np.cumsum(spans)]).astype(np.int64)
        total = int(bases[-1])
        if total + PAD >= 2**31:
            raise ValueError("the edge arena exceeds 2^31 positions")
        self.n_positions = total
        self.caps = caps
        self.bases = [int(b) for b in bases[:-1]]
        self.ends = [int(b) for b in bases[1:]]
        size = total + PAD
        specs = {s.name: s for s in static.conn_fields}
        self.cols = {}
        for name, spec in specs.items():
            dt = torch_dtype(spec.dtype)
            fill = 1 if name == DEAD.name else spec.default
            self.cols[name] = torch.full((size,), fill, dtype=dt, device=device)
        self.slot = torch.full((size,), -1, dtype=torch.int32, device=device)
        self.lives = []
        self.fwd = []
        self.bwd = []
        self.lists: list[SourceLists] = []
        self.dst8 = [None] * nb  # TO_ID is read in full (plx_update_desc.dst8)
        self.blk_dst0 = [None] * nb
        self.fwd_carry = True
        self.bwd_carry = True
        self.dead_in_rows = False
        self.prune_sink = None
        self.t_name = None
        self.t_now = []
        nbits = max(1, int(n).bit_length())
        rows = torch.arange(n, dtype=torch.int32, device=device)
        for b, bucket in enumerate(conns):
            base, cap = self.bases[b], caps[b]
            dead = bucket[DEAD.name]
            live_list, nlive = k.compact(cap, 1, dead)  # PLX_FLAG_U8_ZERO: live slots, ascending
            dead_list, _ = k.compact(cap, 0, dead)  # PLX_FLAG_U8: dead slots, ascending
            live = int(nlive.item())
            self.lives.append(live)
            # Live slots by (destination, slot): a stable sort of the ascending
            # list. Only the live part moves: the step never writes a slot that
            # is dead at layout time, so the dead part keeps fill values and
            # is not written back.
            lv = live_list[:live].clone()
            k.sort(lv, live, [(0, nbits, bucket[TO_ID.name], None)], tag="relayout")
            for name in specs:
                col = bucket[name]
                _lib.check(k.lib.plx_gather_col(live, None, lv.data_ptr(), col.data_ptr(),
                                                self.cols[name][base:].data_ptr(), col.element_size(), k.s),
                           "plx_gather_col")
            self.slot[base : base + live] = lv
            self.slot[base + live : base + cap] = dead_list[: cap - live]
            # Forward rows: every unit; row u owns its in-edges' run.
            fptr = torch.empty(n + 1, dtype=torch.int32, device=device)
            _lib.check(k.lib.plx_sorted_starts(live, self.cols[TO_ID.name][base:].data_ptr(), n, fptr.data_ptr(),
                                               k.s), "plx_sorted_starts")
            self.fwd.append(ForwardRows(n, rows, fptr + base))
            # Backward lists: live slots by (source, slot) -> their positions.
            sl = live_list[:live].clone()
            k.sort(sl, live, [(0, nbits, bucket[FROM_ID.name], None)], tag="relayout")
            pos_of_slot = torch.zeros(cap, dtype=torch.int32, device=device)
            pos_of_slot[lv.long()] = torch.arange(base, base + live, dtype=torch.int32, device=device)
            pos = torch.full((live + 1,), base, dtype=torch.int32, device=device)
            _lib.check(k.lib.plx_gather_i32(live, None, sl.data_ptr(), pos_of_slot.data_ptr(), pos.data_ptr(), k.s),
                       "plx_gather_i32")
            ldst = torch.zeros(live + 1, dtype=torch.int32, device=device)
            _lib.check(k.lib.plx_gather_i32(live, None, sl.data_ptr(), bucket[TO_ID.name].data_ptr(),
                                            ldst.data_ptr(), k.s), "plx_gather_i32")
            lsrc = torch.zeros(max(live, 1), dtype=torch.int32, device=device)
            _lib.check(k.lib.plx_gather_i32(live, None, sl.data_ptr(), bucket[FROM_ID.name].data_ptr(),
                                            lsrc.data_ptr(), k.s), "plx_gather_i32")
            lptr = torch.empty(n + 1, dtype=torch.int32, device=device)
            _lib.check(k.lib.plx_sorted_starts(live, lsrc.data_ptr(), n, lptr.data_ptr(), k.s), "plx_sorted_starts")
            self.lists.append(SourceLists(lptr, pos, ldst))
        self.top = None
        self.levels_dev = levels

    def src_table(self, b: int) -> tuple[int, int]:
        """No source-value tables: units keep the caller's ids."""
        return 0, 0

    def write_logical(self, conns: tuple[Columns, ...]) -> None:
        """Scatter the live part of every bucket back into its logical slots
        (the slots dead at layout time were never written by the step)."""
        for b, bucket in enumerate(conns):
            base, live = self.bases[b], self.lives[b]
            idx = self.slot[base : base + live].long()
            for name, col in bucket.items():
                col[idx] = self.cols[name][base : base + live]
                if name == self.t_name and self.t_now and self.t_now[b] is not None:
                    col[idx] = self.t_now[b]
