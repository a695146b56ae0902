"""The physical edge arena the kernels stream.

The reference stores each bucket source-major in logical slot order
(builder.py:566-579) and reduces with scatters. For the device the same
edges are laid out once more, per bucket, in one slab:

- positions ``[base_b, base_b + live_b)``: the bucket's live edges sorted by
  (destination, logical slot) -- each destination's in-edges are one
  contiguous run, in slot order, which is the order the reference's
  ``segment_sum`` folds them (sweep.py:113-180);
- positions ``[base_b + live_b, end_b)``: the bucket's dead slots in slot
  order, then padding to a multiple of 4 positions (bucket bases are
  multiples of 4, so every tile and vector load is 16-byte aligned);
- ``slot``: the logical slot of every position, so the reference's logical
  view (and slot-ordered free lists) is recovered exactly.

Forward rows are the destination units of a bucket plus the units the
bucket finalizes (phases.py:1011); each row is a CSR range of positions.

The backward is a transpose reduce (sum into FROM_ID, sweep.py:343-399). The
bucket's positions are cut into tiles of ``tile`` positions; within a tile,
the live edges of each source form one group (listed in a per-tile
source-sorted index, ``sorted_local``), folded on the device in physical
order into one partial per (tile, source). Sources present in more than
``HOT_FRAC`` of the tiles (the Zipf head) get a dense per-tile row of
partials (``nhot`` wide); the others get source-major runs of cold partials.
A source's sum is therefore the fold of its tile partials in tile order, each
tile partial the fold of its terms in (dst, slot) order.

Units are not permuted: unit columns are the state's own tensors.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import torch

from plastax_amd._types import DEAD, FROM_ID, TO_ID, Propagation
from plastax_amd.state import Columns, NetworkStatic, column_to_numpy, torch_dtype

TILE = 8192  # positions per backward tile (multiple of 4, <= 32768)
SUPERBLOCK = 32  # tiles per superblock of the cross-tile fold
HOT_FRAC = 0.125  # a source present in more than this fraction of tiles is hot
MAX_HOT = 8192  # dense hot partials per tile (LDS: 4 B each)
PAD = 256  # slack positions after each slab (vector loads may run past the end)


@dataclasses.dataclass
class ForwardRows:
    """Device CSR of one bucket's forward rows."""

    nrows: int
    rows: torch.Tensor  # int32 [nrows] unit ids
    ptr: torch.Tensor  # int32 [nrows+1] physical positions


@dataclasses.dataclass
class BackwardTiles:
    """Device metadata of one bucket's tiled transpose reduce."""

    base: int
    end: int
    ntiles: int
    fold: bool
    nhot: int = 0
    grp_off: torch.Tensor | None = None  # int32 [ntiles+1]
    grp_se: torch.Tensor | None = None  # int32 (uint32 bits) [groups]
    grp_tgt: torch.Tensor | None = None  # int32 [groups]
    sorted_local: torch.Tensor | None = None  # int16 (uint16 bits) [ntiles*tile]
    hot_partial: torch.Tensor | None = None  # f32 [ntiles*nhot]
    hot_sb: torch.Tensor | None = None  # f32 [nsuperblocks*nhot]
    cold_partial: torch.Tensor | None = None  # f32 [ncold]
    cold_sb: torch.Tensor | None = None  # int16 (uint16 bits) [ncold] superblock ids
    nrows: int = 0
    rows: torch.Tensor | None = None  # int32 [nrows] units finalized here
    row_hot: torch.Tensor | None = None  # int32 [nrows]
    row_cold: torch.Tensor | None = None  # int32 [nrows+1]


def _round_up(n: int, k: int) -> int:
    return -(-n // k) * k


class Arena:
    """Physical slab, forward CSR and backward tiles, on the device."""

    def __init__(
        self,
        static: NetworkStatic,
        units: Columns,
        conns: tuple[Columns, ...],
        device: torch.device,
        *,
        tile: int = TILE,
    ) -> None:
        if tile <= 0 or tile % 4 or tile > 32768:
            raise ValueError("tile must be a positive multiple of 4, at most 32768")
        self.static = static
        self.device = device
        self.tile = tile
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
        host = {name: [column_to_numpy(b[name], specs[name]) for b in conns] for name in specs}
        caps = [int(h.shape[0]) for h in host[DEAD.name]]
        spans = [_round_up(c, 4) for c in caps]
        bases = np.concatenate([[0], np.cumsum(spans)]).astype(np.int64)
        total = int(bases[-1])
        self.n_positions = total
        size = total + PAD
        if size >= 2**31:
            raise ValueError("the edge arena exceeds 2^31 positions")
        self.caps = caps
        self.bases = [int(b) for b in bases[:-1]]
        self.ends = [int(b) for b in bases[1:]]

        phys_slot = np.full(size, -1, dtype=np.int32)
        phys = {name: np.full(size, specs[name].default, dtype=specs[name].dtype) for name in specs}
        phys[DEAD.name][:] = True
        self.lives: list[int] = []
        self.fwd: list[ForwardRows] = []
        self.bwd: list[BackwardTiles] = []
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
            self.fwd.append(ForwardRows(int(rows.size), self._i32(rows), self._i32(ptr)))

            # Backward tiles. A TOPOLOGICAL walk never reduces bucket 0
            # (phases.py:1071-1074): it is only updated.
            fold = self.pipeline or b > 0
            srcs = src[order].astype(np.int64)
            if not self.pipeline and fold and live and not bool((levels[srcs] == b).all()):
                self.bwd_carry = True
            self.bwd.append(self._tiles(b, srcs, fold, levels, n))

        # Rows finalized from the identity before the backward bucket walk:
        # the deepest level (phases.py:1089-1094).
        top = np.zeros(0, dtype=np.int64) if self.pipeline else np.flatnonzero(levels == nb)
        self.top = BackwardTiles(0, 0, 0, False, nrows=int(top.size), rows=self._i32(top))

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

    def _i32(self, a: np.ndarray) -> torch.Tensor:
        return torch.from_numpy(np.ascontiguousarray(np.asarray(a).astype(np.int32))).to(self.device)

    def _tiles(self, b: int, srcs: np.ndarray, fold: bool, levels: np.ndarray, n: int) -> BackwardTiles:
        """Tile metadata of bucket b; ``srcs`` are the live edges' sources in
        physical order."""
        T = self.tile
        base, end = self.bases[b], self.ends[b]
        ntiles = -(-(end - base) // T)
        if not fold:
            return BackwardTiles(base, end, ntiles, False)
        live = int(srcs.size)
        rank = np.arange(live, dtype=np.int64)
        tile_of = rank // T
        # The tile's live edges sorted by (source, physical position).
        o2 = np.lexsort((rank, srcs, tile_of))
        t_sorted = tile_of[o2]
        s_sorted = srcs[o2]
        tile_first = np.searchsorted(t_sorted, np.arange(ntiles + 1), side="left")
        sorted_local = np.zeros(ntiles * T + 4, dtype=np.uint16)
        j_in_tile = np.arange(live, dtype=np.int64) - tile_first[t_sorted]
        sorted_local[t_sorted * T + j_in_tile] = (rank[o2] - t_sorted * T).astype(np.uint16)
        # Groups: runs of one source inside one tile.
        if live:
            brk = np.flatnonzero((np.diff(t_sorted) != 0) | (np.diff(s_sorted) != 0)) + 1
            g_start = np.concatenate([[0], brk])
        else:
            g_start = np.zeros(0, dtype=np.int64)
        g_end = np.concatenate([g_start[1:], [live]]).astype(np.int64)
        g_tile = t_sorted[g_start] if live else g_start
        g_src = s_sorted[g_start] if live else g_start
        g_len = g_end - g_start
        g_st = g_start - tile_first[g_tile] if live else g_start
        # Hot sources: present in more than HOT_FRAC of the tiles.
        presence = np.bincount(g_src, minlength=n) if live else np.zeros(n, np.int64)
        cand = np.flatnonzero(presence > HOT_FRAC * ntiles)
        if cand.size > MAX_HOT:
            keep = np.argsort(-presence[cand], kind="stable")[:MAX_HOT]
            cand = np.sort(cand[keep])
        hot_src = cand
        hot_idx = np.full(n, -1, dtype=np.int64)
        hot_idx[hot_src] = np.arange(hot_src.size)
        nhot = int(hot_src.size)
        is_hot = hot_idx[g_src] >= 0 if live else np.zeros(0, bool)
        # Cold groups: source-major, tile order within a source.
        cold = np.flatnonzero(~is_hot)
        cold_order = cold[np.lexsort((g_tile[cold], g_src[cold]))]
        tgt = np.empty(g_start.size, dtype=np.int64)
        tgt[is_hot] = -1 - hot_idx[g_src[is_hot]]
        tgt[cold_order] = np.arange(cold_order.size)
        cold_count = np.bincount(g_src[cold], minlength=n) if cold.size else np.zeros(n, np.int64)
        # Within a tile, longest groups first (lanes take them round robin).
        g_perm = np.lexsort((-g_len, g_tile)) if live else g_start
        grp_off = np.searchsorted(g_tile[g_perm], np.arange(ntiles + 1), side="left")
        se = (g_st[g_perm].astype(np.uint64) | (g_len[g_perm].astype(np.uint64) << np.uint64(16)))
        # Rows finalized at this bucket: hot sources first (by hot slot, so a
        # wave reads consecutive columns), then every other unit of the level.
        if self.pipeline:
            level_units = np.arange(n, dtype=np.int64)
        else:
            level_units = np.union1d(np.flatnonzero(levels == b), np.unique(srcs)).astype(np.int64)
        others = level_units[hot_idx[level_units] < 0]
        rows = np.concatenate([hot_src, others])
        row_hot = np.concatenate([np.arange(nhot), np.full(others.size, -1)])
        # Cold slots were numbered in (source, tile) order and `others` is in
        # source order (hot sources have no cold groups), so each cold row's
        # run is contiguous and the runs follow the row order.
        counts = np.concatenate([np.zeros(nhot, np.int64), cold_count[others]])
        row_cold = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
        assert int(row_cold[-1]) == cold_order.size
        tgt_final = tgt
        ncold = int(cold_order.size)
        cold_sb = (g_tile[cold_order] // SUPERBLOCK).astype(np.uint16)
        nsb = -(-ntiles // SUPERBLOCK)
        dev = self.device
        return BackwardTiles(
            base,
            end,
            ntiles,
            True,
            nhot=nhot,
            grp_off=self._i32(grp_off),
            grp_se=torch.from_numpy(se.astype(np.uint32).view(np.int32)).to(dev),
            grp_tgt=self._i32(tgt_final[g_perm] if live else tgt),
            sorted_local=torch.from_numpy(sorted_local.view(np.int16)).to(dev),
            hot_partial=torch.zeros(max(ntiles * nhot, 1), dtype=torch.float32, device=dev),
            hot_sb=torch.zeros(max(nsb * nhot, 1), dtype=torch.float32, device=dev),
            cold_partial=torch.zeros(max(ncold, 1), dtype=torch.float32, device=dev),
            cold_sb=torch.from_numpy(
                np.concatenate([cold_sb, np.zeros(1, np.uint16)]).view(np.int16)
            ).to(dev),
            nrows=int(rows.size),
            rows=self._i32(rows),
            row_hot=self._i32(row_hot),
            row_cold=self._i32(row_cold),
        )

    def write_logical(self, conns: tuple[Columns, ...]) -> None:
        """Scatter the physical columns back into the logical buckets."""
        for b, bucket in enumerate(conns):
            base, cap = self.bases[b], self.caps[b]
            idx = self.slot[base : base + cap].long()
            for name, col in bucket.items():
                col[idx] = self.cols[name][base : base + cap]
