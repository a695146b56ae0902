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

After a growth step the arena is rebuilt from the previous one (``prev``)
instead: its live edges that are still live keep their (destination, slot)
and (source, slot) orders, so the new orders are those lists merged with
the slots the claim filled, sorted by the same keys (``plx_merge_index``, a
binary search per element) -- one pass over the columns
(``plx_merge_gather``) instead of two radix sorts of every live edge and a
gather per column. The result equals the full build's entry for entry. The
columns alternate between two buffers, so the positions past the live range
keep the fill values with a write of only the range that stopped being live.
"""

from __future__ import annotations

from typing import Any

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

    def __init__(self, ptr: torch.Tensor, pos: torch.Tensor, dst: torch.Tensor, src: torch.Tensor,
                 slot: torch.Tensor) -> None:
        self.ptr = ptr
        self.pos = pos
        self.dst = dst
        self.src = src  # entry j's FROM_ID (the list key)
        self.slot = slot  # entry j's logical slot (the tiebreak)
        n = int(pos.numel())
        self.weight = torch.empty(n, dtype=torch.float32, device=pos.device)
        self.live = torch.empty(n, dtype=torch.uint8, device=pos.device)


class ChurnArena(Arena):
    """A physical arena built on the device from the logical buckets."""

    churn = True

    def __init__(self, static: NetworkStatic, units: Columns, conns: tuple[Columns, ...],
                 device: torch.device, stream: int, prev: "ChurnArena | None" = None,
                 dead_before: list[torch.Tensor] | None = None, claim_bound: int | None = None) -> None:
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
        levels = units["level"]
        self._unit_levels: np.ndarray | None = None  # read from levels_dev on first use
        self.lvl_start = np.zeros(1, np.int64)
        caps = [int(b[DEAD.name].numel()) for b in conns]
        if prev is not None and getattr(prev, "_consts", None) is not None and prev.static is static \
                and prev.device == device:
            # The identity numbering and the id tables depend only on the net:
            # a rebuild keeps its predecessor's.
            (self.uperm, self.uinv, self.uperm_t, self.uinv_t, self.uperm32, self.uinv32, self.input_ids,
             self.output_ids, self.is_input, rows) = prev._consts
        else:
            ident = np.arange(n, dtype=np.int64)
            self.uperm = ident
            self.uinv = ident
            self.uperm_t = torch.arange(n, dtype=torch.int64, device=device)
            self.uinv_t = self.uperm_t
            self.uperm32 = self.uperm_t.to(torch.int32)
            self.uinv32 = self.uperm32
            self.input_ids = self._i32(np.asarray(static.input_ids, dtype=np.int64))
            self.output_ids = self._i32(np.asarray(static.output_ids, dtype=np.int64))
            is_input = np.zeros(n, dtype=np.uint8)
            if static.input_ids:
                is_input[np.asarray(static.input_ids)] = 1
            self.is_input = torch.from_numpy(is_input).to(device)
            rows = torch.arange(n, dtype=torch.int32, device=device)
        self._consts = (self.uperm, self.uinv, self.uperm_t, self.uinv_t, self.uperm32, self.uinv32,
                        self.input_ids, self.output_ids, self.is_input, rows)
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
        self._fills = {name: (1 if name == DEAD.name else spec.default) for name, spec in specs.items()}
        if prev is not None and (dead_before is None or not self.can_follow(prev, static, caps)):
            prev = None
        if prev is not None and prev._spare is not None:
            # the other buffer: fill values past `extent` in every bucket
            self.cols, self.slot, extent = prev._spare
        else:
            self.cols = {}
            for name, spec in specs.items():
                self.cols[name] = torch.full((size,), self._fills[name], dtype=torch_dtype(spec.dtype), device=device)
            self.slot = torch.full((size,), -1, dtype=torch.int32, device=device)
            extent = [0] * nb
        self._spare = None if prev is None else (prev.cols, prev.slot, prev._extent)
        self.merged = prev is not None
        # Columns written since the logical view was last in step (None: any).
        self._written: set | None = set()
        # Per bucket: lives[b], a host bound on its live count that sizes
        # the launches (the count itself after a full build), and
        # live_dev[b], the count on the device (int32[1]). Positions
        # [live, lives[b]) hold fill values (DEAD 1), so the step reads DEAD
        # in the rows of a merged arena.
        self.lives = []
        self.live_dev: list[torch.Tensor] = []
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
        claimed = None
        if prev is not None and not isinstance(dead_before, (list, tuple)):
            # the claim's list of the slots it filled (grow.ClaimedSlots):
            # each bucket's, ascending, in one launch
            out, counts = dead_before.split(k.lib, k.s)
            claimed = [(out[b], counts[b : b + 1]) for b in range(nb)]
        for b, bucket in enumerate(conns):
            if prev is not None:
                fresh = claimed[b] if claimed is not None else dead_before[b]
                self._merge_bucket(k, b, prev, bucket, specs, nbits, rows, extent[b], fresh, claim_bound)
                continue
            base, cap = self.bases[b], caps[b]
            dead = bucket[DEAD.name]
            live_list, nlive = k.compact(cap, 1, dead)  # PLX_FLAG_U8_ZERO: live slots, ascending
            dead_list, _ = k.compact(cap, 0, dead)  # PLX_FLAG_U8: dead slots, ascending
            live = int(nlive.item())
            self.lives.append(live)
            self.live_dev.append(nlive)
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
            _lib.check(k.lib.plx_sorted_starts(live, None, self.cols[TO_ID.name][base:].data_ptr(), n,
                                               fptr.data_ptr(), k.s), "plx_sorted_starts")
            self.fwd.append(ForwardRows(n, rows, fptr + base))
            # Backward lists: live slots by (source, slot) -> their positions.
            sl = live_list[: max(live, 1)].clone()
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
            _lib.check(k.lib.plx_sorted_starts(live, None, lsrc.data_ptr(), n, lptr.data_ptr(), k.s),
                       "plx_sorted_starts")
            self.lists.append(SourceLists(lptr, pos, ldst, lsrc, sl))
        self._extent = list(self.lives)
        self.top = None
        self.levels_dev = levels
        if self.merged:
            self.dead_in_rows = True  # the fill positions up to each bound are dead
        if prev is not None:
            prev._retire()

    def units_to_physical(self, units: Columns) -> Columns:
        """Units keep the caller's ids: the same columns."""
        return dict(units)

    def units_to_logical(self, units: Columns) -> Columns:
        return dict(units)

    @property
    def unit_levels(self) -> np.ndarray:
        """The units' levels on the host, read from the device on first use
        (only the generic passes' finalize lists need them)."""
        if self._unit_levels is None:
            self._unit_levels = self.levels_dev.cpu().numpy().astype(np.int64)
        return self._unit_levels

    @staticmethod
    def can_follow(prev: "ChurnArena", static: NetworkStatic, caps: list[int]) -> bool:
        """Whether a merged rebuild from ``prev`` applies: the same net and
        bucket capacities, ``prev`` still holding its buffers, and columns of
        1- or 4-byte elements (what plx_merge_gather moves)."""
        return (isinstance(prev, ChurnArena) and prev.static is static and prev.caps == caps
                and prev.cols is not None
                and all(np.dtype(s.dtype).itemsize in (1, 4) for s in static.conn_fields))

    def _retire(self) -> None:
        """This arena's buffers now belong to its successor."""
        self.cols = None
        self.slot = None
        self._spare = None

    def _merge_bucket(self, k, b: int, prev: "ChurnArena", bucket: Columns, specs: dict, nbits: int,
                      rows: torch.Tensor, extent: int, dead_before: torch.Tensor, claim_bound: int | None) -> None:
        """Bucket b laid out from ``prev``'s layout of it (see the module
        docstring): the survivors (prev's live positions whose DEAD is still
        0) merged with the slots the claim turned live (``dead_before``: DEAD
        just before the claim, after the step's prunes were copied back).
        Nothing else changes the logical bucket in between, so these are all
        of its live slots. ``dead_before`` may instead be the claim's own list
        of them: (ascending slots, device count), at most ``claim_bound``.

        The counts stay on the device. The launches are sized by host bounds:
        prev's bound on its live count and ``claim_bound``, a bound on the
        claimed slots (the growth's winner budget; the bucket's capacity
        when not given). Ranks past the live count get fill values (slot -1),
        so every array up to the bound is defined."""
        dev = self.device
        n = self.static.num_units
        base, cap = self.bases[b], self.caps[b]
        old_bound, old_live_d = prev.lives[b], prev.live_dev[b]
        new_bound = cap if claim_bound is None else max(0, min(cap, int(claim_bound)))
        bound = min(cap, old_bound + new_bound)
        lib = k.lib
        if prev.t_name and prev.t_now and prev.t_now[b] is not None and old_bound:
            # Adam's count is one number for prev's live edges (its column
            # was not kept for them): materialise it for the survivors.
            t_col = prev.cols[prev.t_name][base : base + old_bound]
            t_col.masked_fill_(prev.cols[DEAD.name][base : base + old_bound] == 0, float(prev.t_now[b]))
        # Survivors: prev's live positions still live, in (destination, slot) order.
        surv, nsurv_d = k.compact(old_bound, 1, prev.cols[DEAD.name][base:], n_dev=old_live_d)  # PLX_FLAG_U8_ZERO
        # New: the slots the claim filled (a slot that died this step may be
        # among them: its old position is not a survivor), ascending: listed
        # by the claim (a (slots, count) pair), or the slots DEAD shows
        # turned live.
        if isinstance(dead_before, tuple):
            fresh, nnew_d = dead_before
        else:
            claimed = (dead_before != 0) & (bucket[DEAD.name] == 0)
            fresh, nnew_d = k.compact(cap, 0, claimed)  # PLX_FLAG_U8: ascending slots
        live_d = nsurv_d + nnew_d
        self.lives.append(bound)
        self.live_dev.append(live_d)
        by_dst = fresh[: max(new_bound, 1)].clone()
        by_src = fresh[: max(new_bound, 1)].clone()
        k.sort(by_dst, new_bound, [(0, nbits, bucket[TO_ID.name], None)], n_dev=nnew_d, tag="relayout")
        k.sort(by_src, new_bound, [(0, nbits, bucket[FROM_ID.name], None)], n_dev=nnew_d, tag="relayout")
        # Positions: merge by (TO_ID, slot); maps old position / new slot -> new position.
        order = torch.empty(max(bound, 1), dtype=torch.int32, device=dev)
        old_to_new = torch.full((max(old_bound, 1),), -1, dtype=torch.int32, device=dev)
        new_pos = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
        m = _lib.plx_merge_desc()
        _side(m.a, old_bound, old_bound, surv, prev.cols[TO_ID.name][base:], prev.slot[base:], old_to_new, nsurv_d)
        _side(m.b, new_bound, cap, by_dst, bucket[TO_ID.name], None, new_pos, nnew_d)
        m.offset, m.order = base, order.data_ptr()
        _lib.check(lib.plx_merge_index(m, k.s), "plx_merge_index")
        cols = [(prev.cols[name][base:], bucket[name], self.cols[name][base:], bucket[name].element_size(),
                 _fill_bits(self._fills[name], bucket[name])) for name in specs]
        cols.append((prev.slot[base:], None, self.slot[base:], 4, _fill_bits(-1, self.slot)))
        _gather(lib, k.s, bound, order, by_dst, new_bound, old_bound, cap, cols, n_dev=live_d)
        # Past the bound: the columns' fill values where the other buffer had more.
        if extent > bound:
            for name, col in self.cols.items():
                col[base + bound : base + extent].fill_(self._fills[name])
            self.slot[base + bound : base + extent].fill_(-1)
        # Forward rows: every unit; row u owns its in-edges' run.
        fptr = torch.empty(n + 1, dtype=torch.int32, device=dev)
        _lib.check(lib.plx_sorted_starts(bound, live_d.data_ptr(), self.cols[TO_ID.name][base:].data_ptr(), n,
                                         fptr.data_ptr(), k.s), "plx_sorted_starts")
        self.fwd.append(ForwardRows(n, rows, fptr + base))
        # Backward lists: the surviving entries (their positions remapped)
        # merged with the new slots by (FROM_ID, slot). Entries of prev's
        # lists past its live count hold position base; the compaction counts
        # only the first old_live_d entries.
        old = prev.lists[b]
        moved = torch.empty(max(old_bound, 1), dtype=torch.int32, device=dev)
        keep = torch.empty(max(old_bound, 1), dtype=torch.uint8, device=dev)
        # New positions of the list entries: from the few dropped positions
        # and inserted slots (old_to_new read at random only past
        # PLX_REMAP_LDS_MAX of either).
        dropped, ndropped_d = k.compact(old_bound, 0, prev.cols[DEAD.name][base:], n_dev=old_live_d)  # PLX_FLAG_U8
        _lib.check(lib.plx_remap_merged(old_bound, old.pos.data_ptr(), base, old_bound, old_to_new.data_ptr(),
                                        dropped.data_ptr(), ndropped_d.data_ptr(), by_dst.data_ptr(),
                                        nnew_d.data_ptr(), max(new_bound, 1), new_pos.data_ptr(), moved.data_ptr(),
                                        keep.data_ptr(), k.s), "plx_remap_merged")
        lsurv, nlsurv_d = k.compact(old_bound, 0, keep, n_dev=old_live_d)  # PLX_FLAG_U8: surviving entries
        lorder = torch.empty(max(bound, 1), dtype=torch.int32, device=dev)
        m2 = _lib.plx_merge_desc()
        _side(m2.a, old_bound, old_bound, lsurv, old.src, old.slot, None, nlsurv_d)
        _side(m2.b, new_bound, cap, by_src, bucket[FROM_ID.name], None, None, nnew_d)
        m2.offset, m2.order = 0, lorder.data_ptr()
        _lib.check(lib.plx_merge_index(m2, k.s), "plx_merge_index")
        # The gather writes every rank below the bound (fill values past the
        # count), so only the trailing entries (pos base, dst 0) are set here.
        pos = torch.empty(bound + 1, dtype=torch.int32, device=dev)
        ldst = torch.empty(bound + 1, dtype=torch.int32, device=dev)
        pos[bound:].fill_(base)
        ldst[bound:].fill_(0)
        lsrc = torch.empty(bound, dtype=torch.int32, device=dev) if bound else torch.zeros(1, dtype=torch.int32, device=dev)
        lslot = torch.empty(bound, dtype=torch.int32, device=dev) if bound else torch.zeros(1, dtype=torch.int32, device=dev)
        _gather(lib, k.s, bound, lorder, by_src, new_bound, old_bound, cap,
                [(moved, new_pos, pos, 4, base), (old.dst, bucket[TO_ID.name], ldst, 4, 0),
                 (old.src, bucket[FROM_ID.name], lsrc, 4, 0), (old.slot, None, lslot, 4, 0)], n_dev=live_d)
        # (pos past the count keeps base: a valid position for the per-step
        # gather of the list's weights, which runs over the whole bound)
        lptr = torch.empty(n + 1, dtype=torch.int32, device=dev)
        _lib.check(lib.plx_sorted_starts(bound, live_d.data_ptr(), lsrc.data_ptr(), n, lptr.data_ptr(), k.s),
                   "plx_sorted_starts")
        self.lists.append(SourceLists(lptr, pos, ldst, lsrc, lslot))

    def live_counts(self) -> list[int]:
        """Each bucket's live count (a host read; the step itself never
        needs it)."""
        return [int(t.item()) for t in self.live_dev]

    def reanchor(self) -> None:
        """Tighten the host bounds to the live counts. The bounds grow by
        the claim's budget at every merge; a caller that waits on the device
        anyway (reading the flags) calls this, one small read more, so a long
        run's launches stay sized by its counts."""
        if self.live_dev:
            counts = torch.cat([t.reshape(1) for t in self.live_dev]).tolist()
            self.lives = [min(bound, int(c)) for bound, c in zip(self.lives, counts)]

    def _write_kills(self, conns: tuple[Columns, ...], written: set) -> None:
        """Only prunes wrote since the logical view was in step: DEAD went
        from 0 to 1 at the killed edges (every position of the live range
        was live at layout time) and the step count was stamped there, so
        only those positions are copied back."""
        from plastax_amd.grow import Kernels

        k = Kernels(self.device, int(torch.cuda.current_stream(self.device).cuda_stream))
        for b, bucket in enumerate(conns):
            base, live, cap = self.bases[b], self.lives[b], self.caps[b]
            if live == 0:
                continue
            # positions now dead among the live count's (past it: fill values)
            killed, nk = k.compact(live, 0, self.cols[DEAD.name][base:], n_dev=self.live_dev[b])  # PLX_FLAG_U8
            for name in written:
                if name not in bucket:
                    continue
                col = bucket[name]
                _lib.check(k.lib.plx_copy_to_slots(live, nk.data_ptr(), killed.data_ptr(), self.slot[base:].data_ptr(),
                                                   self.cols[name][base:].data_ptr(), col.data_ptr(), cap,
                                                   col.element_size(), k.s), "plx_copy_to_slots")

    def src_table(self, b: int) -> tuple[int, int]:
        """No source-value tables: units keep the caller's ids."""
        return 0, 0

    def wrote(self, columns=None) -> None:
        if columns is None or self._written is None:
            self._written = None
        else:
            self._written |= {c for c in columns if c is not None}

    def write_logical(self, conns: tuple[Columns, ...]) -> None:
        """Scatter the live part of every bucket back into its logical slots
        (the slots dead at layout time were never written by the step): the
        columns a step wrote since the last such copy (a prune: DEAD and the
        step count it stamps), or all of them."""
        written, self._written = self._written, set()
        if written is not None and written <= {DEAD.name, self.t_name}:
            self._write_kills(conns, written)
            return
        from plastax_amd.grow import Kernels

        k = Kernels(self.device, int(torch.cuda.current_stream(self.device).cuda_stream))
        for b, bucket in enumerate(conns):
            base, live, cap = self.bases[b], self.lives[b], self.caps[b]
            if live == 0:
                continue
            # positions [0, live count) to their logical slots (the count on the device)
            every = k.iota(live)
            for name, col in bucket.items():
                if written is not None and name not in written:
                    continue
                vals = self.cols[name][base : base + live]
                if name == self.t_name and self.t_now and self.t_now[b] is not None:
                    # Live edges hold the bucket's count; an edge tombstoned
                    # since the layout keeps the count stamped at its kill.
                    vals = torch.where(self.cols[DEAD.name][base : base + live] != 0, vals,
                                       torch.tensor(self.t_now[b], dtype=vals.dtype, device=vals.device))
                vals = vals.contiguous()
                _lib.check(k.lib.plx_copy_to_slots(live, self.live_dev[b].data_ptr(), every.data_ptr(),
                                                   self.slot[base:].data_ptr(), vals.data_ptr(), col.data_ptr(), cap,
                                                   col.element_size(), k.s), "plx_copy_to_slots")


def _side(side, n: int, limit: int, ids: torch.Tensor, key1: torch.Tensor, key2: torch.Tensor | None,
          out_map: torch.Tensor | None, n_dev: torch.Tensor | None = None) -> None:
    side.n, side.id_limit = int(n), int(limit)
    side.ids, side.key1 = ids.data_ptr(), key1.data_ptr()
    side.key2 = None if key2 is None else key2.data_ptr()
    side.map = None if out_map is None else out_map.data_ptr()
    side.n_dev = None if n_dev is None else n_dev.data_ptr()


def _fill_bits(value: Any, like: torch.Tensor) -> int:
    """The bits of ``value`` in the element type of ``like`` (what
    plx_merge_col.fill holds)."""
    if like.dtype == torch.float32:
        return int(np.float32(value).view(np.uint32))
    if like.element_size() == 1:
        return int(bool(value)) if like.dtype == torch.bool else int(np.asarray(value).astype(np.int64)) & 0xFF
    return int(np.asarray(value).astype(np.int64)) & 0xFFFFFFFF


def _gather(lib, stream: int, n: int, order: torch.Tensor, b_ids: torch.Tensor, nb: int, a_limit: int,
            b_limit: int, cols: list[tuple], n_dev: torch.Tensor | None = None) -> None:
    """out[r] = a[order[r]] or b[b_ids[j]] per column (plx_merge_gather), in
    launches of at most PLX_MERGE_MAX_COLS columns; with ``n_dev`` the ranks
    past the device count get each column's fill value (its fifth entry)."""
    if n == 0:
        return
    step = _lib.PLX_MERGE_MAX_COLS
    for c0 in range(0, len(cols), step):
        g = _lib.plx_merge_gather_desc()
        g.n, g.order, g.b_ids, g.nb = int(n), order.data_ptr(), b_ids.data_ptr(), int(nb)
        g.a_limit, g.b_limit = max(int(a_limit), 1), max(int(b_limit), 1)
        g.n_dev = None if n_dev is None else n_dev.data_ptr()
        part = cols[c0 : c0 + step]
        g.ncols = len(part)
        for j, (a, b, out, nbytes, fill) in enumerate(part):
            g.cols[j].a = a.data_ptr()
            g.cols[j].b = None if b is None else b.data_ptr()
            g.cols[j].out = out.data_ptr()
            g.cols[j].bytes = int(nbytes)
            g.cols[j].fill = int(fill)
        _lib.check(lib.plx_merge_gather(g, stream), "plx_merge_gather")
