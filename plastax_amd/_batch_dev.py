"""The batched step's per-bucket tables built on the device.

The reference builds its per-sample CSR views inside the jitted step
(phases.py:843-934). Here they are built once per arena by the library's
stable radix sort, compactions and CSR starts. Small elementwise steps
(shifts, masks, flags) use torch tensor ops. The only host reads are the
table sizes: row and tile counts, which size the launches that use them.

- ``batch_sources_dev``: a bucket's backward rows and each row's live
  out-edges in logical slot order (``batched.BatchSources``);
- ``batch_tiles_dev``: the batched update's tiles, the edges grouped by
  (destination // 64, source // 64) in position order, groups longer than
  BATCH_TILE_EDGES cut (``plx_batch_tiles``).

Both equal the host builds (``batched.batch_sources_host`` /
``_layout.batch_tiles``) entry for entry; ``tests/test_gpu_batch_tables.py``
checks that.
"""

from __future__ import annotations

from typing import Any

import torch

from plastax_amd import _lib
from plastax_amd._layout import BATCH_TILE_EDGES, BATCH_TILE_UNITS


def _kernels(arena: Any) -> Any:
    from plastax_amd.grow import Kernels
    from plastax_amd.step import _stream

    return Kernels(arena.device, _stream(arena.device))


def _bits(n: int) -> int:
    return max(1, int(n).bit_length())


def batch_sources_dev(arena: Any, b: int) -> Any:
    """Bucket b's backward rows on the device: every unit of level b and
    every source of a live edge, ascending; row r's entries
    ``[ptr[r], ptr[r+1])`` are its live positions sorted by logical slot.
    ``pos`` / ``dst`` carry one trailing entry (base / 0), as the host build."""
    from plastax_amd.batched import BatchSources

    k = _kernels(arena)
    dev = arena.device
    n = int(arena.static.num_units)
    base, live = int(arena.bases[b]), int(arena.lives[b])
    frm = arena.cols["from_id"][base : base + live]
    to = arena.cols["to_id"][base : base + live]
    slot = arena.slot[base : base + live]
    order = k.iota(live)
    if live:
        # (source, logical slot), least significant first
        cap = int(arena.static.level_capacities[b])  # logical slots are below the bucket's capacity
        k.sort(order, live, [(0, _bits(cap), slot, None), (0, _bits(n), frm, None)], tag="batch_sources")
    src_sorted = k.gather(order, frm, live, None) if live else torch.zeros(1, dtype=torch.int32, device=dev)
    dst_sorted = k.gather(order, to, live, None) if live else torch.zeros(1, dtype=torch.int32, device=dev)
    # rows: the level's units and every source (a byte mark per unit)
    mark = torch.zeros(n, dtype=torch.uint8, device=dev)
    if b + 1 < arena.lvl_start.size:
        mark[int(arena.lvl_start[b]) : int(arena.lvl_start[b + 1])] = 1
    if live:
        mark[src_sorted[:live].long()] = 1
    rows, nrows_d = k.compact(n, 0, mark)  # PLX_FLAG_U8: ascending unit ids
    nrows = int(nrows_d.item())  # sizes the backward's launches
    start = torch.zeros(n + 1, dtype=torch.int32, device=dev)
    if live:
        _lib.check(k.lib.plx_sorted_starts(live, None, src_sorted.data_ptr(), n, start.data_ptr(), k.s),
                   "plx_sorted_starts")
    ptr = torch.empty(nrows + 1, dtype=torch.int32, device=dev)
    ptr[:nrows] = start[rows[:nrows].long()]
    ptr[nrows] = live
    pos = torch.full((live + 1,), base, dtype=torch.int32, device=dev)
    pos[:live] += order[:live]
    dst = torch.zeros(live + 1, dtype=torch.int32, device=dev)
    dst[:live] = dst_sorted[:live]
    return BatchSources(nrows, rows[:nrows].clone(), ptr, pos, dst)


def batch_tiles_dev(arena: Any, b: int) -> dict[str, torch.Tensor]:
    """Bucket b's batched-update tiles on the device: ``tile_off`` [ntiles +
    1], ``tile_base`` [2 ntiles] (destination and source base of each tile),
    ``pos`` (live positions in tile order) and ``loc`` (uint16 bits:
    destination offset | source offset << 8), as ``_layout.batch_tiles``."""
    k = _kernels(arena)
    dev = arena.device
    n = int(arena.static.num_units)
    u = BATCH_TILE_UNITS
    shift = u.bit_length() - 1
    assert 1 << shift == u
    base, live = int(arena.bases[b]), int(arena.lives[b])
    if live == 0:
        z = torch.zeros(0, dtype=torch.int32, device=dev)
        return {"tile_off": torch.zeros(1, dtype=torch.int32, device=dev), "tile_base": z, "pos": z,
                "loc": torch.zeros(0, dtype=torch.int16, device=dev)}
    frm = arena.cols["from_id"][base : base + live]
    to = arena.cols["to_id"][base : base + live]
    src_t = (frm >> shift).contiguous()
    dst_t = (to >> shift).contiguous()
    order = k.iota(live)
    # (destination tile, source tile), least significant first; position order within
    tbits = _bits(n >> shift)
    k.sort(order, live, [(0, tbits, src_t, None), (0, tbits, dst_t, None)], tag="batch_tiles")
    o = order[:live].long()
    st, dt = src_t[o], dst_t[o]
    # group starts, then each group cut every BATCH_TILE_EDGES entries
    head = torch.ones(live, dtype=torch.bool, device=dev)
    head[1:] = (st[1:] != st[:-1]) | (dt[1:] != dt[:-1])
    starts, _ = k.compact(live, 0, head.to(torch.uint8))
    group = torch.cumsum(head.to(torch.int32), 0, dtype=torch.int32) - 1
    within = torch.arange(live, dtype=torch.int32, device=dev) - starts[group.long()]
    cut = (within % BATCH_TILE_EDGES) == 0
    tiles, ntiles_d = k.compact(live, 0, cut.to(torch.uint8))
    ntiles = int(ntiles_d.item())  # sizes the update's launch
    tile_off = torch.empty(ntiles + 1, dtype=torch.int32, device=dev)
    tile_off[:ntiles] = tiles[:ntiles]
    tile_off[ntiles] = live
    first = o[tile_off[:ntiles].long()]
    tile_base = torch.stack([(to[first] >> shift) << shift, (frm[first] >> shift) << shift], dim=1).reshape(-1)
    loc = ((to[o] & (u - 1)) | ((frm[o] & (u - 1)) << 8)).to(torch.int16)
    return {"tile_off": tile_off, "tile_base": tile_base.to(torch.int32).contiguous(),
            "pos": order[:live].clone(), "loc": loc.contiguous()}
