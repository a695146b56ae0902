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
bucket's positions are cut into at most ``NSUPER`` superblocks of near-equal
length (one device workgroup each) and each superblock into tiles of at most
``tile`` positions (``tile_partition``). Within a tile, the live edges of each
source form one group (``sorted_rank`` gives every live position its rank in
the tile's (source, position) order, so a group is a run of ranks, and marks
the rank that starts each group), folded on the device in physical order
into one partial per (tile, source); 2-byte descriptors (first rank, length)
list a tile's groups longest first. Sources present in many tiles (the Zipf
head) are hot: taken as the first ids of the bucket's source range, the
workgroup keeps their running sums in LDS and writes one dense row per
superblock (``nhot`` wide); the others get cold partials. A source's sum is
therefore the fold, in superblock order, of its superblock sums, each the
fold in tile order of its tile partials, each tile partial the fold of its
terms in (dst, slot) order. Cold partials are stored in one region per XCD
(the finalize workgroups on XCD x read region x), tile-major inside a region,
each slot a function of the group's first rank and the tile's region table
(``tile_info``), and listed source-major by ``cold_idx``. TO_ID is also kept
as one byte per position over a base per 4,096 positions (``dst_bytes``).

Units are renumbered: the arena fixes a physical unit order (``unit_order``:
by level, then out-degree descending, then unit id), the edge columns and
every kernel work in physical ids, and the device unit columns are kept in
that order (``units_to_physical`` / ``units_to_logical`` convert). So each
bucket's most used sources occupy the first ids of their level: the gathers
of their values hit a few cache lines, and a workgroup can copy them into LDS
as one contiguous slice.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import torch

from plastax_amd._types import DEAD, FROM_ID, TO_ID, Propagation
from plastax_amd.state import Columns, NetworkStatic, column_to_numpy, torch_dtype

TILE = 4096  # positions per backward tile (multiple of 4, <= 4096: one device pass)
NSUPER = 512  # superblocks per bucket at most (device workgroups: 2 per CU)
HOT_PER_SUPER = 0.25  # hot iff present in more than this many tiles per superblock
MAX_HOT = 6128  # hot running sums per workgroup (LDS: 4 B each; the fused kernel's LDS stays within 80 KB)
MAX_TBL = 8192  # source values staged in LDS per workgroup (PLX_MAX_TBL)
PAD = 256  # slack positions after each slab (vector loads may run past the end)
PART_ROWS = 256  # cold finalize: rows per workgroup at most (one per lane)
PART_WIN = 2048  # cold finalize: cold partials staged per window
FIN_HOT_COLS = 16  # hot columns per finalize workgroup (PLX_HOT_COLS)
XCDS = 8  # MI355X dies: workgroup w of a launch runs on XCD w % 8
GROUP_START = 0x8000  # sorted_rank bit: the rank starts a (tile, source) group
LEN_OPEN = 15  # group descriptor length field: 15 or more
DST8_BLOCK = 4096  # positions per one-byte destination block (kDst8Shift)
TILE_INFO = 16  # int32 per tile of tile_info (plx_tile_desc)


def xcd_item(first: int, n: int) -> np.ndarray:
    """The item that each of n consecutive workgroups, the first being
    workgroup ``first`` of its launch, takes (the device's xcd_item): each
    XCD's items are one contiguous range, XCD 0's first."""
    i = np.arange(n, dtype=np.int64)
    r = (np.arange(XCDS) - first) % XCDS
    cnt = np.where(r < n, (n - r + XCDS - 1) // XCDS, 0)
    first_item = np.concatenate([[0], np.cumsum(cnt)[:-1]])
    return first_item[(first + i) % XCDS] + i // XCDS


def dst_bytes(dsts: np.ndarray, span: int) -> tuple[np.ndarray | None, np.ndarray | None]:
    """One-byte destinations of a bucket whose live positions' TO_ID
    (``dsts``, destination-sorted) are given: block k of DST8_BLOCK positions
    has base blk_dst0[k] (its first live destination) and position p holds
    TO_ID - blk_dst0[p // DST8_BLOCK]. None, None where a block spans 256 ids
    or more, or the bucket has no live edge."""
    live = int(dsts.size)
    if not live:
        return None, None
    nblk = -(-span // DST8_BLOCK)
    pos = np.arange(live, dtype=np.int64)
    d0 = np.zeros(nblk, dtype=np.int64)
    firsts = np.arange(0, live, DST8_BLOCK)
    d0[: firsts.size] = dsts[firsts]
    delta = dsts - d0[pos // DST8_BLOCK]
    if int(delta.max()) >= 256:
        return None, None
    d8 = np.zeros(span + 4, dtype=np.uint8)
    d8[:live] = delta
    return d8, d0


BATCH_TILE_UNITS = 64  # destination / source units per batched-update tile (kTileRows)
BATCH_TILE_EDGES = 1024  # edges per batched-update tile at most (kTileEdges)


def batch_tiles(src: np.ndarray, dst: np.ndarray) -> dict[str, np.ndarray]:
    """The batched update's tiles of a bucket whose live positions 0.. have
    sources ``src`` and destinations ``dst`` (physical ids): positions
    grouped by (dst // 64, src // 64), in position order within a group,
    groups of more than BATCH_TILE_EDGES cut into several tiles."""
    u = BATCH_TILE_UNITS
    n = int(src.size)
    src = src.astype(np.int64)
    dst = dst.astype(np.int64)
    key = (dst // u) * (int(src.max(initial=0)) // u + 1) + src // u
    order = np.argsort(key, kind="stable")
    ks = key[order]
    starts = np.flatnonzero(np.diff(ks)) + 1 if n else np.zeros(0, np.int64)
    bounds = np.concatenate([[0], starts, [n]]).astype(np.int64) if n else np.zeros(1, np.int64)
    cuts = [np.arange(lo, hi, BATCH_TILE_EDGES) for lo, hi in zip(bounds[:-1], bounds[1:])]
    tile_off = np.concatenate(cuts + [[n]]).astype(np.int64) if n else np.zeros(1, np.int64)
    first = order[tile_off[:-1]]
    tile_base = np.stack([(dst[first] // u) * u, (src[first] // u) * u], axis=1).reshape(-1)
    loc = ((dst[order] % u) | ((src[order] % u) << 8)).astype(np.uint16)
    sizes = np.diff(tile_off)
    if sizes.size and int(sizes.max()) > BATCH_TILE_EDGES:
        raise ValueError("batch_tiles: a tile holds more than BATCH_TILE_EDGES edges")
    if n and (int((loc & 0xFF).max()) >= u or int((loc >> 8).max()) >= u):
        raise ValueError("batch_tiles: a unit offset falls outside its tile")
    return {"tile_off": tile_off, "tile_base": tile_base, "pos": order.astype(np.int64), "loc": loc}


def cold_row_parts(row_cold: np.ndarray, first: int) -> np.ndarray:
    """Split rows [first, nrows) into workgroups of at most PART_ROWS rows
    and, where rows allow, at most PART_WIN cold partials (one LDS window),
    so no workgroup of the finalize waits on far more windows than another.
    Returns the boundaries [first, ..., nrows]."""
    nrows = row_cold.size - 1
    bounds = [first]
    r = first
    while r < nrows:
        hi = min(r + PART_ROWS, nrows)
        # the most rows from r whose cold runs fit one window (at least one)
        fit = int(np.searchsorted(row_cold, row_cold[r] + PART_WIN, side="right")) - 1
        r = max(r + 1, min(hi, fit))
        bounds.append(r)
    return np.asarray(bounds, dtype=np.int64)


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
    nsuper: int = 0
    tile_pos: torch.Tensor | None = None  # int32 [ntiles+1] tile starts (relative to base)
    super_tile: torch.Tensor | None = None  # int32 [nsuper+1] first tile of each superblock
    nhot: int = 0
    hot_base: int = 0  # hot sources are physical ids [hot_base, hot_base + nhot)
    tile_info: torch.Tensor | None = None  # int32 [ntiles, TILE_INFO] hot ranks, cold regions
    grp_off: torch.Tensor | None = None  # int32 [ntiles+1]
    grp: torch.Tensor | None = None  # int16 (uint16 bits) [groups] first rank | min(len, 15) << 12
    sorted_rank: torch.Tensor | None = None  # int16 (uint16 bits) [span]: rank | GROUP_START
    hot_sb: torch.Tensor | None = None  # f32 [nsuper*nhot]
    cold_partial: torch.Tensor | None = None  # f32 [ncold]
    cold_sb: torch.Tensor | None = None  # int16 (uint16 bits) [ncold] superblock ids
    cold_idx: torch.Tensor | None = None  # int32 [ncold groups] slot, source-major order
    nrows: int = 0
    rows: torch.Tensor | None = None  # int32 [nrows] units finalized here
    row_hot: torch.Tensor | None = None  # int32 [nrows]
    row_cold: torch.Tensor | None = None  # int32 [nrows+1]
    nparts: int = 0
    part_rows: torch.Tensor | None = None  # int32 [nparts+1] cold rows per workgroup
    part_info: torch.Tensor | None = None  # int32 [nparts, 4] (first row, end row, first, end cold entry)


def _round_up(n: int, k: int) -> int:
    return -(-n // k) * k


def unit_order(levels: np.ndarray, live_src: np.ndarray) -> np.ndarray:
    """The physical unit order: units sorted by level, then by out-degree
    (live edges leaving the unit) descending, then by id. Returns ``uperm``:
    physical index -> unit id."""
    n = levels.size
    outdeg = np.bincount(live_src.astype(np.int64), minlength=n)
    return np.lexsort((np.arange(n), -outdeg, levels.astype(np.int64)))


def tile_partition(span: int, tile: int, nsuper_max: int = NSUPER) -> tuple[np.ndarray, np.ndarray]:
    """Cut positions [0, span) (span a multiple of 4) into superblocks and
    tiles: ``nsuper = min(nsuper_max, ceil(span / tile))`` superblocks, the
    k-th starting at ``(k * span // nsuper)`` rounded down to a multiple of 4,
    each cut into tiles of ``tile`` positions (the last one shorter). Returns
    (tile_pos [ntiles+1], super_tile [nsuper+1]): tile t covers
    [tile_pos[t], tile_pos[t+1]); superblock k owns tiles
    [super_tile[k], super_tile[k+1])."""
    if span % 4 or tile % 4 or tile <= 0:
        raise ValueError("tile_partition: span and tile must be multiples of 4")
    if span == 0:
        return np.zeros(1, np.int64), np.zeros(1, np.int64)
    nsuper = min(nsuper_max, -(-span // tile))
    starts = [(k * span // nsuper) & ~3 for k in range(nsuper)] + [span]
    tile_pos: list[int] = []
    super_tile: list[int] = []
    for k in range(nsuper):
        lo, hi = starts[k], starts[k + 1]
        if hi <= lo:
            raise AssertionError("tile_partition: empty superblock")
        super_tile.append(len(tile_pos))
        tile_pos.extend(range(lo, hi, tile))
    super_tile.append(len(tile_pos))
    tile_pos.append(span)
    return np.asarray(tile_pos, np.int64), np.asarray(super_tile, np.int64)


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
        nsuper: int = NSUPER,
    ) -> None:
        if tile <= 0 or tile % 4 or tile > 4096:
            raise ValueError("tile must be a positive multiple of 4, at most 4096")
        if not 1 <= nsuper <= 65535:
            raise ValueError("nsuper must be in [1, 65535]")
        self.static = static
        self.device = device
        self.tile = tile
        self.nsuper = nsuper
        n = static.num_units
        nb = len(conns)
        self.num_buckets = nb
        self.pipeline = static.propagation is Propagation.PIPELINE
        specs = {s.name: s for s in static.conn_fields}
        host = {name: [column_to_numpy(b[name], specs[name]) for b in conns] for name in specs}
        # Physical unit order; from here on every unit id is physical.
        levels_l = units["level"].cpu().numpy().astype(np.int64)
        live_src = np.concatenate(
            [h[~d] for h, d in zip(host[FROM_ID.name], host[DEAD.name])] or [np.zeros(0, np.int32)]
        )
        self.uperm = unit_order(levels_l, live_src)
        self.uinv = np.empty(n, dtype=np.int64)
        self.uinv[self.uperm] = np.arange(n)
        self.uperm_t = torch.from_numpy(self.uperm).to(device)
        self.uinv_t = torch.from_numpy(self.uinv).to(device)
        # int32 copies for the kernels that translate ids (physical <-> caller's).
        self.uperm32 = self.uperm_t.to(torch.int32)
        self.uinv32 = self.uinv_t.to(torch.int32)
        for name in (FROM_ID.name, TO_ID.name):
            host[name] = [self.uinv[np.clip(h, 0, n - 1)].astype(np.int32) for h in host[name]]
        levels = levels_l[self.uperm]
        self.unit_levels = levels  # levels in the physical unit order
        is_input = np.zeros(n, dtype=bool)
        if static.input_ids:
            is_input[self.uinv[np.asarray(static.input_ids)]] = True
        pruned = units.get("pruned")
        live_unit = np.ones(n, dtype=bool) if pruned is None else pruned.cpu().numpy()[self.uperm] == 0
        # First physical id of every level (level l is [lvl_start[l], lvl_start[l+1])).
        self.lvl_start = np.searchsorted(levels, np.arange(int(levels.max(initial=0)) + 2))
        # Per-arena device constants in physical ids.
        self.input_ids = self._i32(self.uinv[np.asarray(static.input_ids, dtype=np.int64)])
        self.output_ids = self._i32(self.uinv[np.asarray(static.output_ids, dtype=np.int64)])
        self.is_input = torch.from_numpy(is_input.astype(np.uint8)).to(device)
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
        # One-byte destinations per bucket (None where a block spans >= 256 ids).
        self.dst8: list[torch.Tensor | None] = []
        self.blk_dst0: list[torch.Tensor | None] = []
        self.fwd: list[ForwardRows] = []
        self.bwd: list[BackwardTiles] = []
        self.fwd_carry = False
        self.bwd_carry = False
        # Live positions come first in every bucket, so no forward row range
        # holds a tombstone until one is set in place after this build.
        self.dead_in_rows = False
        self.prune_sink: torch.Tensor | None = None  # the fused forward's tombstones (plastax_amd.fusion)
        # Adam's step count when every live edge of a bucket holds the same
        # one (per bucket; None: the per-edge column is authoritative).
        self.t_name: str | None = None
        self.t_now: list[float | None] = []
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
            self.bwd.append(self._tiles(b, srcs, dsts, fold, levels, n))
            d8, d0 = dst_bytes(dsts, self.ends[b] - base)
            self.dst8.append(None if d8 is None else torch.from_numpy(d8).to(device))
            self.blk_dst0.append(None if d0 is None else self._i32(d0))

        # Rows finalized from the identity before the backward bucket walk:
        # the deepest level (phases.py:1089-1094).
        top = np.zeros(0, dtype=np.int64) if self.pipeline else np.flatnonzero(levels == nb)
        top_parts = np.minimum(np.arange(0, top.size + PART_ROWS, PART_ROWS), top.size)
        top_parts = np.unique(top_parts) if top.size else np.zeros(1, np.int64)
        self.top = BackwardTiles(0, 0, 0, False, nrows=int(top.size), rows=self._i32(top),
                                 nparts=top_parts.size - 1, part_rows=self._i32(top_parts))

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

    def _tiles(self, b: int, srcs: np.ndarray, dsts: np.ndarray, fold: bool, levels: np.ndarray,
               n: int) -> BackwardTiles:
        """Tile metadata of bucket b; ``srcs`` / ``dsts`` are the live edges'
        sources and destinations in physical order."""
        T = self.tile
        base, end = self.bases[b], self.ends[b]
        tile_pos, super_tile = tile_partition(end - base, T, self.nsuper)
        ntiles = tile_pos.size - 1
        nsuper = super_tile.size - 1
        tables = dict(nsuper=nsuper, tile_pos=self._i32(tile_pos), super_tile=self._i32(super_tile))
        if not fold:
            return BackwardTiles(base, end, ntiles, False, **tables)
        live = int(srcs.size)
        rank = np.arange(live, dtype=np.int64)
        tile_of = np.searchsorted(tile_pos, rank, side="right") - 1
        sb_of_tile = np.searchsorted(super_tile, np.arange(ntiles), side="right") - 1
        # The tile's live edges sorted by (source, physical position).
        o2 = np.lexsort((rank, srcs, tile_of))
        t_sorted = tile_of[o2]
        s_sorted = srcs[o2]
        tile_first = np.searchsorted(t_sorted, np.arange(ntiles + 1), side="left")
        j_in_tile = np.arange(live, dtype=np.int64) - tile_first[t_sorted]
        # Groups: runs of one source inside one tile; sorted_rank carries each
        # position's rank (low 12 bits) and whether that rank starts a group.
        if live:
            brk = np.flatnonzero((np.diff(t_sorted) != 0) | (np.diff(s_sorted) != 0)) + 1
            g_start = np.concatenate([[0], brk])
        else:
            g_start = np.zeros(0, dtype=np.int64)
        starts = np.zeros(live, dtype=np.int64)
        starts[g_start] = GROUP_START
        sorted_rank = np.zeros(int(tile_pos[-1]) + 4, dtype=np.uint16)
        sorted_rank[rank[o2]] = (j_in_tile | starts).astype(np.uint16)
        g_tile = t_sorted[g_start] if live else g_start
        g_src = s_sorted[g_start] if live else g_start
        g_st = j_in_tile[g_start] if live else g_start
        g_end = np.concatenate([g_start[1:], [live]]).astype(np.int64)
        g_len = g_end - g_start
        # Descriptors: within a tile, longest groups first (lanes take them
        # round robin), each its first rank and min(length, 15).
        g_perm = np.lexsort((-g_len, g_tile)) if live else g_start
        grp_off = np.searchsorted(g_tile[g_perm], np.arange(ntiles + 1), side="left")
        grp = (g_st[g_perm] | (np.minimum(g_len[g_perm], LEN_OPEN) << 12)).astype(np.uint16)
        # Hot sources: a dense superblock row costs 8 B per superblock (write
        # and read), a cold partial about as much as a scattered 4-byte store
        # plus its read per tile present: as many hot sources as there are
        # sources present in more than HOT_PER_SUPER tiles per superblock,
        # taken as the first ids of the bucket's source range (units are
        # numbered busiest first), so a source's hot index is its id less
        # hot_base and the hot ranks of a tile are one range.
        if self.pipeline:
            hb, he = 0, n
        elif b + 1 < self.lvl_start.size:
            hb, he = int(self.lvl_start[b]), int(self.lvl_start[b + 1])
        else:
            hb, he = 0, 0
        presence = np.bincount(g_src, minlength=n) if live else np.zeros(n, np.int64)
        nhot = int(min(np.count_nonzero(presence > max(1.0, HOT_PER_SUPER * nsuper)), MAX_HOT, he - hb))
        hot_src = np.arange(hb, hb + nhot, dtype=np.int64)
        is_hot = np.zeros(n, dtype=bool)
        is_hot[hot_src] = True
        # Rows finalized at this bucket: hot sources first (by hot index, so a
        # wave reads consecutive columns), then every other unit of the level.
        if self.pipeline:
            level_units = np.arange(n, dtype=np.int64)
        else:
            level_units = np.union1d(np.flatnonzero(levels == b), np.unique(srcs)).astype(np.int64)
        others = level_units[~is_hot[level_units]]
        rows = np.concatenate([hot_src, others])
        row_hot = np.concatenate([np.arange(nhot), np.full(others.size, -1)])
        # Cold groups in (source, tile) order; `others` is in source order
        # (hot sources have no cold groups), so each cold row's entries are
        # one run and the runs follow the row order.
        cold = np.flatnonzero(~is_hot[g_src]) if live else g_start
        cold_order = cold[np.lexsort((g_tile[cold], g_src[cold]))]
        cold_count = np.bincount(g_src[cold], minlength=n) if cold.size else np.zeros(n, np.int64)
        counts = np.concatenate([np.zeros(nhot, np.int64), cold_count[others]])
        row_cold = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
        assert int(row_cold[-1]) == cold_order.size
        cold_sb = sb_of_tile[g_tile[cold_order]].astype(np.uint16)
        parts = cold_row_parts(row_cold, nhot)
        # Each tile's hot ranks: [hlo, hhi) (sources below hot_base sort first).
        hlo = np.bincount(t_sorted[s_sorted < hb], minlength=ntiles)[:ntiles] if live else np.zeros(ntiles, np.int64)
        hcnt = np.bincount(t_sorted[is_hot[s_sorted]], minlength=ntiles)[:ntiles] if live else np.zeros(ntiles, np.int64)
        hhi = hlo + hcnt
        # Cold slots: one region per XCD, holding the partials that the
        # finalize workgroups on that XCD read, so each XCD's L2 fetches only
        # its region. The finalize hands the cold parts to its workgroups by
        # xcd_item, so a part's region grows with the part, hence with the
        # source id, and within a tile the cold ranks of a region are one
        # range. A cold group starting at rank r gets the slot o[x] + c, with
        # c its rank among the tile's cold ranks (hot ranks skipped) and x its
        # region: inside a region, slots are tile-major and a tile's are one
        # run (holes where a cold group spans several ranks).
        nparts = parts.size - 1
        hot_wgs = -(-nhot // FIN_HOT_COLS) if nhot and nsuper else 0
        region_of_part = np.zeros(max(nparts, 1), dtype=np.int64)
        if nparts:
            region_of_part[xcd_item(hot_wgs, nparts)] = (hot_wgs + np.arange(nparts)) % XCDS
        row_of = np.full(n, -1, dtype=np.int64)
        row_of[rows] = np.arange(rows.size)
        cold_e = np.flatnonzero(~is_hot[s_sorted]) if live else g_start
        e_tile = t_sorted[cold_e]
        e_region = region_of_part[np.searchsorted(parts, row_of[s_sorted[cold_e]], side="right") - 1]
        e_c = j_in_tile[cold_e] - np.where(j_in_tile[cold_e] >= hhi[e_tile], hcnt[e_tile], 0)
        cnt = np.bincount(e_tile * XCDS + e_region, minlength=ntiles * XCDS).reshape(ntiles, XCDS)
        bnd = np.concatenate([np.zeros((ntiles, 1), np.int64), np.cumsum(cnt, axis=1)], axis=1)
        assert ((bnd[e_tile, e_region] <= e_c) & (e_c < bnd[e_tile, e_region + 1])).all()
        totals = cnt.sum(axis=0)
        rbase = np.concatenate([[0], np.cumsum(totals)[:-1]])
        cum = np.cumsum(cnt, axis=0) - cnt
        off = rbase[None, :] + cum - bnd[:, :XCDS]
        ncold = int(cnt.sum())
        g_region = region_of_part[np.searchsorted(parts, row_of[g_src[cold_order]], side="right") - 1]
        gt = g_tile[cold_order]
        gst = g_st[cold_order]
        g_c = gst - np.where(gst >= hhi[gt], hcnt[gt], 0)
        cold_idx = off[gt, g_region] + g_c
        info = np.zeros((max(ntiles, 1), TILE_INFO), dtype=np.int64)
        if ntiles:
            info[:ntiles, 0] = hlo | (hhi << 16)
            info[:ntiles, 1:8] = bnd[:, 1:8]
            info[:ntiles, 8:] = off
        dev = self.device
        return BackwardTiles(
            base,
            end,
            ntiles,
            True,
            nhot=nhot,
            hot_base=hb,
            tile_info=torch.from_numpy(info.reshape(-1).astype(np.uint32).view(np.int32)).to(dev),
            grp_off=self._i32(grp_off),
            grp=torch.from_numpy(np.concatenate([grp, np.zeros(1, np.uint16)]).view(np.int16)).to(dev),
            # (one spare entry each: a bucket without live edges still gets
            # real, if unused, tables)
            cold_idx=self._i32(np.concatenate([cold_idx, np.zeros(1, np.int64)])),
            sorted_rank=torch.from_numpy(sorted_rank.view(np.int16)).to(dev),
            hot_sb=torch.zeros(max(nsuper * nhot, 1), dtype=torch.float32, device=dev),
            cold_partial=torch.zeros(max(ncold, 1), dtype=torch.float32, device=dev),
            cold_sb=torch.from_numpy(
                np.concatenate([cold_sb, np.zeros(1, np.uint16)]).view(np.int16)
            ).to(dev),
            nrows=int(rows.size),
            rows=self._i32(rows),
            row_hot=self._i32(row_hot),
            row_cold=self._i32(row_cold),
            nparts=nparts,
            part_rows=self._i32(parts),
            part_info=self._i32(np.stack([parts[:-1], parts[1:], row_cold[parts[:-1]], row_cold[parts[1:]]],
                                         axis=1).reshape(-1) if parts.size > 1 else np.zeros(4, np.int64)),
            **tables,
        )

    def write_logical(self, conns: tuple[Columns, ...]) -> None:
        """Scatter the physical columns back into the logical buckets (unit
        ids mapped back to the caller's numbering)."""
        for b, bucket in enumerate(conns):
            base, cap = self.bases[b], self.caps[b]
            idx = self.slot[base : base + cap].long()
            for name, col in bucket.items():
                vals = self.cols[name][base : base + cap]
                if name in (FROM_ID.name, TO_ID.name):
                    vals = self.uperm_t[vals.long()].to(col.dtype)
                col[idx] = vals
                if name == self.t_name and self.t_now and self.t_now[b] is not None:
                    # Live edges hold the bucket's count; an edge tombstoned
                    # since the layout keeps the count stamped at its kill.
                    live = slice(base, base + self.lives[b])
                    col[idx[: self.lives[b]]] = torch.where(self.cols[DEAD.name][live] != 0, self.cols[name][live],
                                                            self.t_now[b])

    def wrote(self, columns: Any = None) -> None:
        """A step wrote ``columns`` (None: any) of this arena; write_logical
        copies every column back regardless."""

    def init_uniform_t(self, t_name: str) -> None:
        """Adam's per-edge step count: where every live edge of a bucket holds
        the same integer count below 2^23 (each step adds exactly 1.0 to
        every live edge, so they stay equal), keep it as one number per
        bucket; the kernels then neither read nor write that column."""
        self.t_name = t_name
        col = self.cols[t_name]
        self.t_now = []
        for b in range(self.num_buckets):
            live = col[self.bases[b] : self.bases[b] + self.lives[b]]
            t = None
            if live.numel():
                lo, hi = float(live.min()), float(live.max())
                if lo == hi and lo == int(lo) and 0.0 <= lo < 2.0**23:
                    t = lo
            self.t_now.append(t)

    def drop_uniform_t(self) -> None:
        """Keep Adam's step count per edge from here on: write the bucket's
        count into the column of its live edges (a tombstone keeps the count
        stamped at its kill) and let the kernels read and advance the column
        (a captured graph cannot carry a count the host advances)."""
        if not (self.t_name and self.t_now):
            return
        col = self.cols[self.t_name]
        for b, t in enumerate(self.t_now):
            if t is None:
                continue
            live = slice(self.bases[b], self.bases[b] + self.lives[b])
            col[live].masked_fill_(self.cols[DEAD.name][live] == 0, float(t))
            self.t_now[b] = None

    def logical_ids(self) -> dict[str, torch.Tensor]:
        """FROM_ID and TO_ID of every position in the caller's numbering (the
        slab holds arena unit ids), for site programs that read them: built
        on first use (4 bytes per position each) and kept with the arena,
        whose ids never change in place. Ids outside [0, num_units) are
        clamped first, as the kernels' own id translation does."""
        cached = getattr(self, "_logical_ids", None)
        if cached is None:
            n = self.static.num_units
            cached = {name: self.uperm32[self.cols[name].clamp(0, n - 1).long()]
                      for name in (FROM_ID.name, TO_ID.name)}
            self._logical_ids = cached
        return cached

    def stamp_target(self, b: int) -> tuple[torch.Tensor | None, float]:
        """(column from bucket b's base, value) that a kill in bucket b
        stamps: Adam's step-count column and the bucket's count while every
        live edge shares it (the column is not kept for live edges then), so
        a tombstoned edge keeps the count it died with; (None, 0) otherwise."""
        if self.t_name and self.t_now and self.t_now[b] is not None:
            return self.cols[self.t_name][self.bases[b] :], float(self.t_now[b])
        return None, 0.0

    def live_end(self, b: int) -> int:
        """End of bucket b's live positions (live edges come first)."""
        return self.bases[b] + self.lives[b]

    def src_table(self, b: int) -> tuple[int, int]:
        """(base, len) of bucket b's source-value table: its busiest sources,
        the first physical ids of the sources' level (all units for a
        PIPELINE bucket), at most PLX_MAX_TBL of them."""
        if self.pipeline:
            return 0, min(MAX_TBL, self.static.num_units)
        if b + 1 >= self.lvl_start.size:
            return 0, 0
        lo, hi = int(self.lvl_start[b]), int(self.lvl_start[b + 1])
        return lo, min(MAX_TBL, hi - lo)

    def units_to_physical(self, units: Columns) -> Columns:
        """Unit columns in the caller's numbering -> physical order."""
        return {k: v.index_select(0, self.uperm_t) for k, v in units.items()}

    def units_to_logical(self, units: Columns) -> Columns:
        """Physical unit columns -> the caller's numbering."""
        return {k: v.index_select(0, self.uinv_t) for k, v in units.items()}
