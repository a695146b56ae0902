"""The physical edge arena the kernels stream.

The reference stores each bucket source-major in logical slot order
(builder.py:566-579) and reduces with scatters. For the device the same
edges are laid out once more, per bucket, in one slab:

- positions ``[base_b, base_b + live_b)``: the bucket's live edges sorted by
  (destination, logical slot) -- each destination's in-edges are one
  contiguous run, in slot order, which is the order the reference's
  ``segment_sum`` folds them (sweep.py:113-180);
- positions ``[base_b + live_b, base_b + cap_b)``: the bucket's dead slots in
  slot order;
- ``slot``: the logical slot of every position, so the reference's logical
  view (and slot-ordered free lists) can be recovered exactly.

Forward rows are the destination units of a bucket plus the units the
bucket finalizes (phases.py:1011); each row is a CSR range of positions.
The backward reads a source-sorted mirror of each bucket: for every live
edge in (source, slot) order its physical position (``sperm``) and its
destination (``sdst``). A source with more than ``PIECE`` out-edges is split
into pieces of at most ``PIECE`` consecutive terms (the items a lane folds);
the piece sums are folded in order by the finalize kernel.

Units are not permuted: unit columns are the state's own tensors.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import torch

from plastax_amd._types import DEAD, FROM_ID, TO_ID, Propagation
from plastax_amd.state import Columns, NetworkStatic, column_to_numpy, torch_dtype

PIECE = 256  # terms per backward item
PAD = 256  # slack positions after each slab (vector loads may run past the end)


@dataclasses.dataclass
class BucketRows:
    """Device CSR of one bucket's forward or backward rows."""

    nrows: int
    rows: torch.Tensor  # int32 [nrows] unit ids
    ptr: torch.Tensor | None  # int32 [nrows+1] (forward: positions; backward: items)
    nitems: int = 0
    item_ptr: torch.Tensor | None = None  # int32 [nitems+1] mirror positions
    item_base: int = 0  # offset of this bucket's items in the item_sum scratch


def _round_up(n: int, k: int) -> int:
    return -(-n // k) * k


class Arena:
    """Physical slab + forward CSR + backward mirror, on the device."""

    def __init__(
        self,
        static: NetworkStatic,
        units: Columns,
        conns: tuple[Columns, ...],
        device: torch.device,
    ) -> None:
        self.static = static
        self.device = device
        n = static.num_units
        nb = len(conns)
        self.num_buckets = nb
        self.pipeline = static.propagation is Propagation.PIPELINE
        levels = units["level"].cpu().numpy().astype(np.int64)
        is_input = np.zeros(n, dtype=bool)
        if static.input_ids:
            is_input[np.asarray(static.input_ids)] = True
        pruned = units.get("pruned")
        live_unit = np.ones(n, dtype=bool) if pruned is None else pruned.cpu().numpy() == 0
        specs = {s.name: s for s in static.conn_fields}
        host = {
            name: [column_to_numpy(b[name], specs[name]) for b in conns] for name in specs
        }
        caps = [int(h.shape[0]) for h in host[DEAD.name]]
        bases = np.concatenate([[0], np.cumsum(caps)]).astype(np.int64)
        total = int(bases[-1])
        self.total = total
        self.n_positions = _round_up(total, 4)  # the update kernel's range
        size = self.n_positions + PAD
        if size >= 2**31:
            raise ValueError("the edge arena exceeds 2^31 positions")
        self.caps = caps
        self.bases = [int(b) for b in bases[:-1]]

        phys_slot = np.full(size, -1, dtype=np.int32)
        phys = {name: np.full(size, specs[name].default, dtype=specs[name].dtype) for name in specs}
        phys[DEAD.name][:] = True
        self.lives: list[int] = []
        fwd_rows_h: list[tuple[np.ndarray, np.ndarray]] = []
        mirrors: list[tuple[np.ndarray, np.ndarray, np.ndarray]] = []
        self.fwd_carry = False
        self.bwd_carry = False
        for b in range(nb):
            base, cap = self.bases[b], caps[b]
            dead = host[DEAD.name][b]
            src = host[FROM_ID.name][b]
            dst = host[TO_ID.name][b]
            live_idx = np.flatnonzero(~dead)
            dead_idx = np.flatnonzero(dead)
            # Stable sort of the live slots by destination: ties keep slot order.
            order = live_idx[np.argsort(dst[live_idx], kind="stable")]
            slots = np.concatenate([order, dead_idx]).astype(np.int32)
            phys_slot[base : base + cap] = slots
            for name in specs:
                phys[name][base : base + cap] = host[name][b][slots]
            live = int(order.size)
            self.lives.append(live)
            pos_of_slot = np.empty(cap, dtype=np.int64)
            pos_of_slot[slots] = base + np.arange(cap)

            # Forward rows: destinations of this bucket and the units it
            # finalizes (phases.py:1011; sweep.py:328-338 for PIPELINE).
            dsts = dst[order].astype(np.int64)
            if self.pipeline:
                fin = np.flatnonzero(~is_input & live_unit)
            else:
                fin = np.flatnonzero((levels == b + 1) & ~is_input & live_unit)
                fin_of_dst = (levels[dsts] == b + 1) & ~is_input[dsts] & live_unit[dsts]
                if live and not bool(fin_of_dst.all()):
                    self.fwd_carry = True
            rows = np.union1d(np.unique(dsts), fin).astype(np.int64)
            lo = np.searchsorted(dsts, rows, side="left")
            ptr = np.concatenate([lo, [live]]).astype(np.int64) + base
            fwd_rows_h.append((rows.astype(np.int32), ptr.astype(np.int32)))

            # Backward mirror (sweep.py:343-399): live edges in (src, slot) order.
            # A TOPOLOGICAL walk never reduces bucket 0 (phases.py:1071-1074).
            mirrored = live_idx if (self.pipeline or b > 0) else live_idx[:0]
            by_src = mirrored[np.argsort(src[mirrored], kind="stable")]
            srcs = src[by_src].astype(np.int64)
            sperm = pos_of_slot[by_src].astype(np.int32)
            sdst = dst[by_src].astype(np.int32)
            if self.pipeline:
                brows = np.arange(n, dtype=np.int64)
            else:
                brows = np.union1d(np.flatnonzero(levels == b), np.unique(srcs)).astype(np.int64)
                if live and not bool((levels[srcs] == b).all()):
                    self.bwd_carry = True
            mirrors.append((brows, srcs, np.stack([sperm, sdst])))

        # Assemble the mirror slab and the backward items.
        mtotal = sum(int(m[1].size) for m in mirrors)
        msize = _round_up(mtotal, 4) + PAD
        sperm_all = np.zeros(msize, dtype=np.int32)
        sdst_all = np.full(msize, -1, dtype=np.int32)
        mbase = 0
        item_base = 0
        self.bwd: list[BucketRows] = []
        self.fwd: list[BucketRows] = []
        for b in range(nb):
            brows, srcs, sp_sd = mirrors[b]
            m = int(srcs.size)
            sperm_all[mbase : mbase + m] = sp_sd[0]
            sdst_all[mbase : mbase + m] = sp_sd[1]
            lo = np.searchsorted(srcs, brows, side="left")
            hi = np.searchsorted(srcs, brows, side="right")
            counts = hi - lo
            npieces = -(-counts // PIECE)
            row_item = np.concatenate([[0], np.cumsum(npieces)]).astype(np.int64)
            nitems = int(row_item[-1])
            # item k of row r starts at lo[r] + j * PIECE
            item_start = np.empty(nitems + 1, dtype=np.int64)
            if nitems:
                owner = np.repeat(np.arange(brows.size), npieces)
                j = np.arange(nitems) - row_item[owner]
                item_start[:nitems] = lo[owner] + j * PIECE
            item_start[nitems] = m
            item_start += mbase
            self.bwd.append(
                BucketRows(
                    nrows=int(brows.size),
                    rows=self._i32(brows),
                    ptr=self._i32(row_item + item_base),
                    nitems=nitems,
                    item_ptr=self._i32(item_start),
                    item_base=item_base,
                )
            )
            item_base += nitems
            mbase += m
            rows, ptr = fwd_rows_h[b]
            self.fwd.append(BucketRows(nrows=int(rows.size), rows=self._i32(rows), ptr=self._i32(ptr)))
        self.total_items = item_base
        # Rows finalized from the identity before the backward bucket walk:
        # the deepest level (phases.py:1089-1094).
        if self.pipeline:
            top = np.zeros(0, dtype=np.int64)
        else:
            top = np.flatnonzero(levels == nb)
        self.top = BucketRows(nrows=int(top.size), rows=self._i32(top), ptr=None)

        self.slot = torch.from_numpy(phys_slot).to(device)
        self.cols: Columns = {}
        for name, spec in specs.items():
            arr = phys[name]
            if arr.dtype == np.bool_:
                arr = arr.view(np.uint8)
            elif arr.dtype == np.uint32:
                arr = arr.view(np.int32)
            self.cols[name] = torch.from_numpy(np.ascontiguousarray(arr)).to(device)
            assert self.cols[name].dtype == torch_dtype(spec.dtype)
        self.sperm = torch.from_numpy(sperm_all).to(device)
        self.sdst = torch.from_numpy(sdst_all).to(device)
        self.item_sum = torch.zeros(max(self.total_items, 1), dtype=torch.float32, device=device)

    def _i32(self, a: np.ndarray) -> torch.Tensor:
        return torch.from_numpy(np.ascontiguousarray(a.astype(np.int32))).to(self.device)

    def write_logical(self, conns: tuple[Columns, ...]) -> None:
        """Scatter the physical columns back into the logical buckets."""
        for b, bucket in enumerate(conns):
            base, cap = self.bases[b], self.caps[b]
            idx = self.slot[base : base + cap].long()
            for name, col in bucket.items():
                col[idx] = self.cols[name][base : base + cap]
