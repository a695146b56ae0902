"""The tiled arena built on the device.

The same arena as ``_layout.Arena`` (same physical unit order, slab, forward
rows, tiles, groups, hot / cold partials: the tables are equal entry for
entry), built from the logical buckets without taking the edge columns to
the host:

- unit order: out-degrees by an integer histogram of the live sources
  (``plx_count_ids``), then a stable radix sort by (level, -out-degree, id);
- per bucket: the live slots by ordered compaction, stably sorted by
  physical destination (``plx_sort``), every column gathered into the slab;
- forward rows and their ranges from the destinations' histogram;
- the tiles' transpose tables with ``plx_tile_build`` (one workgroup per tile
  sorts it by (source, position) in LDS; a counting pass, then the tables),
  the cold groups by a stable sort by source and ``plx_cold_slots``.

The host sees only unit-sized vectors (levels, the unit order, per-unit
counts) and per-tile counts, which fix the table sizes and the finalize's
cold-row parts (``cold_row_parts``, a sequential greedy cut).
"""

from __future__ import annotations

import numpy as np
import torch

from plastax_amd import _lib
from plastax_amd._layout import (
    DST8_BLOCK,
    FIN_HOT_COLS,
    GROUP_START,  # noqa: F401 - the rank flag plx_tile_build sets (0x8000)
    HOT_PER_SUPER,
    LEN_OPEN,  # noqa: F401 - the descriptor length cap plx_tile_build applies
    MAX_HOT,
    NSUPER,
    PAD,
    PART_ROWS,
    TILE,
    TILE_INFO,
    XCDS,
    Arena,
    BackwardTiles,
    ForwardRows,
    _round_up,
    cold_row_parts,
    tile_partition,
    xcd_item,
)
from plastax_amd._types import DEAD, FROM_ID, TO_ID, Propagation
from plastax_amd.state import Columns, NetworkStatic, torch_dtype


def _bits(n: int) -> int:
    return max(1, int(n).bit_length())


class DeviceArena(Arena):
    """``Arena`` with its edge-sized work done on the device."""

    def __init__(self, static: NetworkStatic, units: Columns, conns: tuple[Columns, ...], device: torch.device,
                 stream: int, *, tile: int = TILE, nsuper: int = NSUPER) -> None:
        from plastax_amd.grow import Kernels

        if tile <= 0 or tile % 4 or tile > 4096:
            raise ValueError("tile must be a positive multiple of 4, at most 4096")
        if not 1 <= nsuper <= 65535:
            raise ValueError("nsuper must be in [1, 65535]")
        self.static = static
        self.device = device
        self.tile = tile
        self.nsuper = nsuper
        self._k = k = Kernels(device, stream)
        lib = k.lib
        n = static.num_units
        nb = len(conns)
        self.num_buckets = nb
        self.pipeline = static.propagation is Propagation.PIPELINE
        specs = {s.name: s for s in static.conn_fields}

        # Physical unit order: level, out-degree descending, id.
        levels_l = units["level"].cpu().numpy().astype(np.int64)
        outdeg = torch.zeros(n, dtype=torch.int32, device=device)
        for bucket in conns:
            cap = int(bucket[DEAD.name].numel())
            _lib.check(lib.plx_count_ids(cap, bucket[FROM_ID.name].data_ptr(), bucket[DEAD.name].data_ptr(), n,
                                         outdeg.data_ptr(), k.s), "plx_count_ids")
        deg_key = (torch.full_like(outdeg, 0x7FFFFFFF) - outdeg).contiguous()
        lvl_dev = torch.from_numpy(levels_l.astype(np.int32)).to(device)
        order = torch.arange(n, dtype=torch.int32, device=device)
        k.sort(order, n, [(0, 31, deg_key, None), (0, _bits(int(levels_l.max(initial=0))), lvl_dev, None)],
               tag="layout")
        self.uperm = order.cpu().numpy().astype(np.int64)
        self.uinv = np.empty(n, dtype=np.int64)
        self.uinv[self.uperm] = np.arange(n)
        self.uperm_t = torch.from_numpy(self.uperm).to(device)
        self.uinv_t = torch.from_numpy(self.uinv).to(device)
        self.uperm32 = self.uperm_t.to(torch.int32)
        self.uinv32 = self.uinv_t.to(torch.int32)
        levels = levels_l[self.uperm]
        self.unit_levels = levels
        is_input = np.zeros(n, dtype=bool)
        if static.input_ids:
            is_input[self.uinv[np.asarray(static.input_ids)]] = True
        pruned = units.get("pruned")
        live_unit = np.ones(n, dtype=bool) if pruned is None else pruned.cpu().numpy()[self.uperm] == 0
        self.lvl_start = np.searchsorted(levels, np.arange(int(levels.max(initial=0)) + 2))
        self.input_ids = self._i32(self.uinv[np.asarray(static.input_ids, dtype=np.int64)])
        self.output_ids = self._i32(self.uinv[np.asarray(static.output_ids, dtype=np.int64)])
        self.is_input = torch.from_numpy(is_input.astype(np.uint8)).to(device)
        caps = [int(b[DEAD.name].numel()) for b in conns]
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
        self.cols = {}
        for name, spec in specs.items():
            fill = 1 if name == DEAD.name else spec.default
            self.cols[name] = torch.full((size,), fill, dtype=torch_dtype(spec.dtype), device=device)
        self.slot = torch.full((size,), -1, dtype=torch.int32, device=device)
        self.lives = []
        self.dst8 = []
        self.blk_dst0 = []
        self.fwd = []
        self.bwd = []
        self.fwd_carry = False
        self.bwd_carry = False
        self.dead_in_rows = False
        self.prune_sink = None
        self.t_name = None
        self.t_now = []
        nbits = _bits(n)
        for b, bucket in enumerate(conns):
            base, cap = self.bases[b], caps[b]
            dead = bucket[DEAD.name]
            live_list, nlive = k.compact(cap, 1, dead)  # live slots, ascending
            dead_list, _ = k.compact(cap, 0, dead)
            live = int(nlive.item())
            self.lives.append(live)
            phys = {}
            for name in (FROM_ID.name, TO_ID.name):
                ids = bucket[name].clamp(0, n - 1).to(torch.int32).contiguous()
                phys[name] = k.gather(ids, self.uinv32, cap, None)
            # Live slots by (physical destination, slot): a stable sort of the ascending list.
            lv = live_list[:live].contiguous()
            k.sort(lv, live, [(0, nbits, phys[TO_ID.name], None)], tag="layout")
            slots = torch.cat([lv, dead_list[: cap - live]]).contiguous()
            self.slot[base : base + cap] = slots
            for name, spec in specs.items():
                col = phys[name] if name in phys else bucket[name]
                _lib.check(lib.plx_gather_col(cap, None, slots.data_ptr(), col.data_ptr(),
                                              self.cols[name][base:].data_ptr(), col.element_size(), k.s),
                           "plx_gather_col")
            dsts = self.cols[TO_ID.name][base : base + live]
            srcs = self.cols[FROM_ID.name][base : base + live]
            cnt_dst = torch.zeros(n, dtype=torch.int32, device=device)
            cnt_src = torch.zeros(n, dtype=torch.int32, device=device)
            if live:
                _lib.check(lib.plx_count_ids(live, dsts.data_ptr(), None, n, cnt_dst.data_ptr(), k.s), "plx_count_ids")
                _lib.check(lib.plx_count_ids(live, srcs.data_ptr(), None, n, cnt_src.data_ptr(), k.s), "plx_count_ids")
            in_deg = cnt_dst.cpu().numpy().astype(np.int64)
            out_deg = cnt_src.cpu().numpy().astype(np.int64)
            start = np.concatenate([[0], np.cumsum(in_deg)])

            # Forward rows (phases.py:1011; sweep.py:328-338 for PIPELINE).
            if self.pipeline:
                fin = ~is_input & live_unit
            else:
                fin = (levels == b + 1) & ~is_input & live_unit
                if live and bool(((in_deg > 0) & ~fin).any()):
                    self.fwd_carry = True
            rows = np.flatnonzero((in_deg > 0) | fin).astype(np.int64)
            ptr = np.concatenate([start[rows], [live]]).astype(np.int64) + base
            self.fwd.append(ForwardRows(int(rows.size), self._i32(rows), self._i32(ptr)))

            fold = self.pipeline or b > 0
            if not self.pipeline and fold and live and bool(((out_deg > 0) & (levels != b)).any()):
                self.bwd_carry = True
            self.bwd.append(self._tiles_dev(b, srcs, live, out_deg, fold, levels, n))

            # One-byte destinations: block k's base is its first live destination.
            span = self.ends[b] - base
            if live:
                firsts = np.arange(0, live, DST8_BLOCK)
                lasts = np.minimum(firsts + DST8_BLOCK, live) - 1
                d0_first = np.searchsorted(start, firsts, side="right") - 1
                d0_last = np.searchsorted(start, lasts, side="right") - 1
                ok = bool((d0_last - d0_first).max() < 256)
            else:
                ok = False
            if ok:
                nblk = -(-span // DST8_BLOCK)
                d0 = np.zeros(nblk, dtype=np.int64)
                d0[: firsts.size] = d0_first
                d0_t = self._i32(d0)
                rel = torch.arange(live, dtype=torch.int64, device=device) >> 12
                d8 = torch.zeros(span + 4, dtype=torch.uint8, device=device)
                d8[:live] = (dsts - d0_t[rel]).to(torch.uint8)
                self.dst8.append(d8)
                self.blk_dst0.append(d0_t)
            else:
                self.dst8.append(None)
                self.blk_dst0.append(None)

        top = np.zeros(0, dtype=np.int64) if self.pipeline else np.flatnonzero(levels == nb)
        top_parts = np.minimum(np.arange(0, top.size + PART_ROWS, PART_ROWS), top.size)
        top_parts = np.unique(top_parts) if top.size else np.zeros(1, np.int64)
        self.top = BackwardTiles(0, 0, 0, False, nrows=int(top.size), rows=self._i32(top),
                                 nparts=top_parts.size - 1, part_rows=self._i32(top_parts))

    def _tiles_dev(self, b: int, srcs: torch.Tensor, live: int, out_deg: np.ndarray, fold: bool,
                   levels: np.ndarray, n: int) -> BackwardTiles:
        """Bucket b's tile tables (``Arena._tiles``, on the device)."""
        k = self._k
        lib = k.lib
        dev = self.device
        T = self.tile
        base, end = self.bases[b], self.ends[b]
        tile_pos, super_tile = tile_partition(end - base, T, self.nsuper)
        ntiles = tile_pos.size - 1
        nsuper = super_tile.size - 1
        tp = self._i32(tile_pos)
        tables = dict(nsuper=nsuper, tile_pos=tp, super_tile=self._i32(super_tile))
        if not fold:
            return BackwardTiles(base, end, ntiles, False, **tables)
        # Pass 0: groups per tile and tiles per source.
        d = _lib.plx_tile_build_desc()
        d.ntiles, d.live = ntiles, live
        d.tile_pos = tp.data_ptr()
        d.src = srcs.data_ptr() if live else None
        presence = torch.zeros(n, dtype=torch.int32, device=dev)
        ngroups = torch.zeros(max(ntiles, 1), dtype=torch.int32, device=dev)
        d.pass_ = 0
        d.ngroups, d.presence = ngroups.data_ptr(), presence.data_ptr()
        _lib.check(lib.plx_tile_build(d, k.s), "plx_tile_build")
        pres = presence.cpu().numpy().astype(np.int64)
        ng = ngroups.cpu().numpy().astype(np.int64)[:ntiles]
        if (ng < 0).any():
            raise ValueError(f"plx_tile_build: tile {int(np.flatnonzero(ng < 0)[0])} spans more than "
                             "4096 positions")
        grp_off = np.concatenate([[0], np.cumsum(ng)]).astype(np.int64)
        total_groups = int(grp_off[-1])

        if self.pipeline:
            hb, he = 0, n
        elif b + 1 < self.lvl_start.size:
            hb, he = int(self.lvl_start[b]), int(self.lvl_start[b + 1])
        else:
            hb, he = 0, 0
        nhot = int(min(np.count_nonzero(pres > max(1.0, HOT_PER_SUPER * nsuper)), MAX_HOT, he - hb))
        hot_src = np.arange(hb, hb + nhot, dtype=np.int64)
        is_hot = np.zeros(n, dtype=bool)
        is_hot[hot_src] = True
        if self.pipeline:
            level_units = np.arange(n, dtype=np.int64)
        else:
            level_units = np.flatnonzero((levels == b) | (out_deg > 0)).astype(np.int64)
        others = level_units[~is_hot[level_units]]
        rows = np.concatenate([hot_src, others])
        row_hot = np.concatenate([np.arange(nhot), np.full(others.size, -1)])
        counts = np.concatenate([np.zeros(nhot, np.int64), pres[others]])
        row_cold = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
        parts = cold_row_parts(row_cold, nhot)
        nparts = parts.size - 1
        hot_wgs = -(-nhot // FIN_HOT_COLS) if nhot and nsuper else 0
        region_of_part = np.zeros(max(nparts, 1), dtype=np.int64)
        if nparts:
            region_of_part[xcd_item(hot_wgs, nparts)] = (hot_wgs + np.arange(nparts)) % XCDS
        region = np.zeros(n, dtype=np.int8)
        if others.size and nparts:
            r_of = np.arange(nhot, rows.size)
            region[others] = region_of_part[np.searchsorted(parts, r_of, side="right") - 1].astype(np.int8)
        region_t = torch.from_numpy(region).to(dev)

        # Pass 1: the tables.
        span = end - base
        sorted_rank = torch.zeros(span + 4, dtype=torch.int16, device=dev)
        grp = torch.zeros(total_groups + 1, dtype=torch.int16, device=dev)
        g_src = torch.zeros(max(total_groups, 1), dtype=torch.int32, device=dev)
        g_st = torch.zeros_like(g_src)
        g_tile = torch.zeros_like(g_src)
        hl = torch.zeros(max(2 * ntiles, 2), dtype=torch.int32, device=dev)
        cnt = torch.zeros(max(8 * ntiles, 8), dtype=torch.int32, device=dev)
        grp_off_t = self._i32(grp_off)
        d.pass_ = 1
        d.hot_base, d.nhot = hb, nhot
        d.grp_off, d.region = grp_off_t.data_ptr(), region_t.data_ptr()
        d.sorted_rank, d.grp = sorted_rank.data_ptr(), grp.data_ptr()
        d.g_src, d.g_st, d.g_tile = g_src.data_ptr(), g_st.data_ptr(), g_tile.data_ptr()
        d.hl, d.cnt = hl.data_ptr(), cnt.data_ptr()
        _lib.check(lib.plx_tile_build(d, k.s), "plx_tile_build")
        hl_h = hl.cpu().numpy().astype(np.int64)[: 2 * ntiles].reshape(ntiles, 2)
        cnt_h = cnt.cpu().numpy().astype(np.int64)[: 8 * ntiles].reshape(ntiles, XCDS)
        hlo, hcnt = hl_h[:, 0], hl_h[:, 1]
        hhi = hlo + hcnt
        bnd = np.concatenate([np.zeros((ntiles, 1), np.int64), np.cumsum(cnt_h, axis=1)], axis=1)
        totals = cnt_h.sum(axis=0)
        rbase = np.concatenate([[0], np.cumsum(totals)[:-1]])
        cum = np.cumsum(cnt_h, axis=0) - cnt_h
        off = rbase[None, :] + cum - bnd[:, :XCDS]
        ncold = int(cnt_h.sum())
        info = np.zeros((max(ntiles, 1), TILE_INFO), dtype=np.int64)
        if ntiles:
            info[:ntiles, 0] = hlo | (hhi << 16)
            info[:ntiles, 1:8] = bnd[:, 1:8]
            info[:ntiles, 8:] = off

        # Cold groups by (source, tile) and their slots.
        ncg = int(row_cold[-1])
        cold_idx = torch.zeros(ncg + 1, dtype=torch.int32, device=dev)
        cold_sb = torch.zeros(ncg + 1, dtype=torch.int16, device=dev)
        if total_groups:
            flag = ((g_src[:total_groups] < hb) | (g_src[:total_groups] >= hb + nhot)).to(torch.uint8)
            cold, ncold_dev = k.compact(total_groups, 0, flag)
            k.sort(cold, total_groups, [(0, _bits(n), g_src, None)], n_dev=ncold_dev, tag="layout")
            sb_of_tile = np.searchsorted(super_tile, np.arange(ntiles), side="right") - 1
            off_t = self._i32(off.reshape(-1))
            sb_t = self._i32(sb_of_tile)
            _lib.check(lib.plx_cold_slots(total_groups, ncold_dev.data_ptr(), cold.data_ptr(), g_src.data_ptr(),
                                          g_st.data_ptr(), g_tile.data_ptr(), hl.data_ptr(), off_t.data_ptr(),
                                          region_t.data_ptr(), sb_t.data_ptr(), cold_idx.data_ptr(),
                                          cold_sb.data_ptr(), k.s), "plx_cold_slots")
        return BackwardTiles(
            base,
            end,
            ntiles,
            True,
            nhot=nhot,
            hot_base=hb,
            tile_info=torch.from_numpy(info.reshape(-1).astype(np.uint32).view(np.int32)).to(dev),
            grp_off=grp_off_t,
            grp=grp,
            cold_idx=cold_idx,
            sorted_rank=sorted_rank,
            hot_sb=torch.zeros(max(nsuper * nhot, 1), dtype=torch.float32, device=dev),
            cold_partial=torch.zeros(max(ncold, 1), dtype=torch.float32, device=dev),
            cold_sb=cold_sb,
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
