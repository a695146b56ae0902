"""The physical arena's metadata, checked on the CPU.

Every index the kernels dereference is bounds-checked here, and a numpy
emulation of the device's tiled backward fold (same groups, same order, float32
arithmetic) must reproduce the oracle's tiled fold bit for bit -- so a layout
bug shows up on the CPU before any kernel reads the metadata.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import nets
import plastax_amd as px
from plastax_amd import _layout, synth


def _sum_map(field: str):
    """The linear sum_ map over ``field`` as the oracle's pass plans state it."""
    import types

    return types.SimpleNamespace(field=field, monoid=0, w_const=None, x_const=None)


def _arena(net, e, tile, nsuper=_layout.NSUPER, **kw):
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cpu", **kw)
    arena = _layout.Arena(static, state.units, state.conns, torch.device("cpu"), tile=tile,
                          nsuper=nsuper)
    return static, state, arena


def _np(t):
    return t.numpy()


def _check_arena(static, state, arena) -> None:
    size = arena.n_positions + _layout.PAD
    assert arena.cols["weight"].numel() == size
    src = _np(arena.cols["from_id"])
    dst = _np(arena.cols["to_id"])
    dead = _np(arena.cols["dead"]).astype(bool)
    slot = _np(arena.slot)
    n = static.num_units
    assert src.min() >= 0 and src.max() < n and dst.min() >= 0 and dst.max() < n
    for b, (base, end, cap) in enumerate(zip(arena.bases, arena.ends, arena.caps)):
        assert base % 4 == 0 and end % 4 == 0 and end - base >= cap
        assert sorted(slot[base : base + cap].tolist()) == list(range(cap))
        assert (slot[base + cap : end] == -1).all() and dead[base + cap : end].all()
        live = arena.lives[b]
        assert not dead[base : base + live].any() and dead[base + live : base + cap].all()
        # forward CSR
        fr = arena.fwd[b]
        rows, ptr = _np(fr.rows), _np(fr.ptr)
        assert (np.diff(rows) > 0).all() and (np.diff(ptr) >= 0).all()
        assert ptr[0] == base and ptr[-1] == base + live
        for r in range(rows.size):
            assert (dst[ptr[r] : ptr[r + 1]] == rows[r]).all()
        # destination-sorted with slot order inside a destination
        d_live = dst[base : base + live]
        s_live = slot[base : base + live]
        key = d_live.astype(np.int64) * (cap + 1) + s_live
        assert (np.diff(key) > 0).all()


def _emulate_fold(arena, b, g_logical: np.ndarray):
    """The device's superblock/tile fold + partials fold, in numpy float32.
    Takes the grad field in the caller's unit numbering; returns sums keyed by
    the caller's unit ids."""
    g_field = g_logical[arena.uperm]  # the device's unit order
    bt = arena.bwd[b]
    T = arena.tile
    w = _np(arena.cols["weight"])
    dst = _np(arena.cols["to_id"])
    src = _np(arena.cols["from_id"])
    dead = _np(arena.cols["dead"]).astype(bool)
    rank = _np(bt.sorted_rank).view(np.uint16).astype(np.int64)
    info = _np(bt.tile_info).reshape(-1, _layout.TILE_INFO).astype(np.int64)
    goff = _np(bt.grp_off)
    grp = _np(bt.grp).view(np.uint16).astype(np.int64)
    tile_pos = _np(bt.tile_pos)
    super_tile = _np(bt.super_tile)
    nhot, nsuper, hb = bt.nhot, bt.nsuper, bt.hot_base
    assert tile_pos[0] == 0 and tile_pos[-1] == bt.end - bt.base and (np.diff(tile_pos) > 0).all()
    assert (np.diff(tile_pos) <= T).all() and (tile_pos % 4 == 0).all()
    assert super_tile[0] == 0 and super_tile[-1] == bt.ntiles and (np.diff(super_tile) > 0).all()
    live_end = bt.base + arena.lives[b]
    if arena.dst8[b] is not None:  # the one-byte destinations are exact below live_end
        d8 = _np(arena.dst8[b]).astype(np.int64)
        d0 = _np(arena.blk_dst0[b]).astype(np.int64)
        pos = np.arange(arena.lives[b])
        assert (d0[pos // _layout.DST8_BLOCK] + d8[pos] == dst[bt.base + pos]).all()
    hot_sb = np.zeros(nsuper * nhot, np.float32)
    cold = np.zeros(_np(bt.cold_partial).size, np.float32)
    written = np.zeros(cold.size, bool)
    seen = np.zeros(bt.end - bt.base, np.int64)
    for sb in range(nsuper):
        run = np.zeros(nhot, np.float32)
        for k in range(super_tile[sb], super_tile[sb + 1]):
            t0 = bt.base + tile_pos[k]
            n = tile_pos[k + 1] - tile_pos[k]
            nr = int(min(n, max(0, live_end - t0)))
            # the ranked positions, placed at their rank with the device's tag
            at = np.full(nr, -1, np.int64)
            tag = np.zeros(nr, np.int64)
            buf = np.zeros(nr, np.float32)
            for p in range(nr):
                raw = int(rank[tile_pos[k] + p])
                r = raw & 0x0FFF
                assert r < nr and at[r] == -1
                e = t0 + p
                at[r] = e
                h = int(src[e]) - hb
                tag[r] = (raw & _layout.GROUP_START) | (h if 0 <= h < nhot else 0)
                buf[r] = np.float32(0.0) if dead[e] else np.float32(w[e] * g_field[dst[e]])
            # (source, position) order, and the start bits mark source changes
            for r in range(1, nr):
                a0, a1 = at[r - 1], at[r]
                assert (src[a0], a0) < (src[a1], a1)
                assert bool(tag[r] & _layout.GROUP_START) == (src[a0] != src[a1])
            assert nr == 0 or tag[0] & _layout.GROUP_START
            hlo, hhi = int(info[k, 0] & 0xFFFF), int(info[k, 0] >> 16)
            assert all((hlo <= r < hhi) == (0 <= src[at[r]] - hb < nhot) for r in range(nr))
            bnd = info[k, 1:8]
            off = info[k, 8:16]
            touched = set()
            for gi in range(goff[k], goff[k + 1]):
                st, ln = int(grp[gi] & 0x0FFF), int(grp[gi] >> 12)
                assert tag[st] & _layout.GROUP_START and 1 <= ln <= _layout.LEN_OPEN
                if ln == _layout.LEN_OPEN:  # at least 15: the run ends at the next start
                    ln = next((j for j in range(st + 1, nr) if tag[j] & _layout.GROUP_START), nr) - st
                    assert ln >= _layout.LEN_OPEN
                assert st + ln <= nr
                assert all(not tag[j] & _layout.GROUP_START for j in range(st + 1, st + ln))
                assert st + ln == nr or tag[st + ln] & _layout.GROUP_START
                v = np.float32(0.0)
                for j in range(st, st + ln):
                    seen[at[j] - bt.base] += 1
                    v = np.float32(v + buf[j])
                if hlo <= st < hhi:
                    h = int(tag[st] & 0x7FFF)
                    assert h == src[at[st]] - hb and h not in touched  # one writer per tile
                    touched.add(h)
                    run[h] = np.float32(run[h] + v)
                else:
                    c = st - (hhi - hlo if st >= hhi else 0)
                    slot = int(off[sum(int(c >= x) for x in bnd)] + c)
                    assert 0 <= slot < cold.size and not written[slot]
                    written[slot] = True
                    cold[slot] = v
            # longest groups first
            lens = []
            for gi in range(goff[k], goff[k + 1]):
                st = int(grp[gi] & 0x0FFF)
                lens.append(next((j for j in range(st + 1, nr) if tag[j] & _layout.GROUP_START), nr) - st)
            assert lens == sorted(lens, reverse=True)
        hot_sb[sb * nhot : (sb + 1) * nhot] = run
    live = arena.lives[b]
    assert (seen[:live] == 1).all() and (seen[live:] == 0).all()
    rows = _np(bt.rows)
    row_hot = _np(bt.row_hot)
    row_cold = _np(bt.row_cold)
    # one slot per cold rank (groups spanning several ranks leave holes)
    assert row_cold[0] == 0 and (np.diff(row_cold) >= 0).all() and row_cold[-1] <= cold.size
    cold_sb = _np(bt.cold_sb).view(np.uint16)
    cold_idx = _np(bt.cold_idx)
    ncold = row_cold[-1]
    assert np.unique(cold_idx[:ncold]).size == ncold and written[cold_idx[:ncold]].all()  # every cold group's slot
    # the finalize kernel relies on hot rows coming first, in column order,
    # and on the cold workgroups covering the other rows, 256 at most each
    assert (row_hot[:nhot] == np.arange(nhot)).all() and (row_hot[nhot:] == -1).all()
    assert (rows[:nhot] == hb + np.arange(nhot)).all()  # hot index = id - hot_base
    parts = _np(bt.part_rows)
    assert bt.nparts == parts.size - 1 and parts[0] == nhot and parts[-1] == rows.size
    assert (np.diff(parts) > 0).all() and (np.diff(parts) <= _layout.PART_ROWS).all()
    one_row = np.diff(parts) == 1
    assert (np.diff(row_cold[parts])[~one_row] <= _layout.PART_WIN).all()
    out = {}
    for r in range(rows.size):
        s = np.float32(0.0)
        if row_hot[r] >= 0:
            for sb in range(nsuper):
                s = np.float32(s + hot_sb[sb * nhot + row_hot[r]])
        else:
            j0, j1 = row_cold[r], row_cold[r + 1]
            if j0 < j1:
                cur, q = cold_sb[j0], np.float32(0.0)
                for j in range(j0, j1):
                    if cold_sb[j] != cur:
                        s, q, cur = np.float32(s + q), np.float32(0.0), cold_sb[j]
                    q = np.float32(q + cold[cold_idx[j]])
                s = np.float32(s + q)
        out[int(arena.uperm[rows[r]])] = s
    return out


@pytest.mark.parametrize("tile,nsuper,hub", [(64, 512, False), (256, 512, False), (64, 7, False), (96, 3, False),
                                              (128, 512, True), (128, 3, True)])
def test_tiled_fold_emulation_matches_oracle_exactly(oracle, tile: int, nsuper: int, hub: bool) -> None:
    e = nets.hub_edges(4) if hub else synth.c2_topological(seed=2, scale=512, layers=4)
    net = nets.make_trained_net("L", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.sgd(0.1, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state, arena = _arena(net, e, tile, nsuper=nsuper)
    _check_arena(static, state, arena)
    if nsuper < 512:
        assert any(np.diff(_np(arena.bwd[b].super_tile)).max() > 1 for b in range(1, arena.num_buckets))
    o = nets.oracle_for(oracle, net, static, state, tile=tile, nsuper=nsuper)
    rng = np.random.default_rng(0)
    g = rng.standard_normal(static.num_units).astype(np.float32)
    o.units["grad_pre_act"][:] = g
    assert any(arena.bwd[b].nhot > 0 for b in range(1, arena.num_buckets))
    # one-byte destinations on the Zipf nets; the hub net's wide bucket keeps four
    assert all(d is not None for d in arena.dst8) if not hub else any(d is None for d in arena.dst8)
    if hub:  # groups of 15 or more ranks (their end is found from the start bits)
        assert any(((_np(arena.bwd[b].grp).view(np.uint16) >> 12) == _layout.LEN_OPEN).any()
                   for b in range(1, arena.num_buckets))
    for b in range(1, arena.num_buckets):
        got = _emulate_fold(arena, b, g)
        want = o._reduce_bwd(b, _sum_map("grad_pre_act"))
        for u, v in got.items():
            assert np.float32(v).view(np.uint32) == want[u].view(np.uint32), (b, u, v, want[u])


def test_pipeline_arena_and_fold(oracle) -> None:
    e = synth.c1_pipeline(0, num_units=256, num_edges=2048)
    net = nets.make_trained_net("LP", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.sgd(0.1, nets.GRAD_PRE_ACT), px.Propagation.PIPELINE)
    static, state, arena = _arena(net, e, 128)
    _check_arena(static, state, arena)
    o = nets.oracle_for(oracle, net, static, state, tile=128)
    g = np.random.default_rng(1).standard_normal(static.num_units).astype(np.float32)
    o.units["grad_pre_act"][:] = g
    got = _emulate_fold(arena, 0, g)
    want = o._reduce_bwd(0, _sum_map("grad_pre_act"))
    assert len(got) == static.num_units  # every unit is a PIPELINE backward row
    for u, v in got.items():
        assert np.float32(v).view(np.uint32) == want[u].view(np.uint32)


def test_arena_with_dead_slots_and_headroom() -> None:
    e = synth.c2_topological(seed=4, scale=1024, layers=3)
    net = nets.make_trained_net("LH", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.adam(1e-3, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cpu", capacity_headroom=0.5,
        capacity_align=7)
    # kill a scattered third of the live slots
    for bucket in state.conns:
        dead = bucket["dead"]
        live = torch.nonzero(dead == 0).flatten()
        dead[live[::3]] = 1
    arena = _layout.Arena(static, state.units, state.conns, torch.device("cpu"), tile=96)
    _check_arena(static, state, arena)
    g = np.random.default_rng(2).standard_normal(static.num_units).astype(np.float32)
    for b in range(1, arena.num_buckets):
        _emulate_fold(arena, b, g)


def test_write_logical_round_trips() -> None:
    e = synth.c2_topological(seed=6, scale=1024, layers=3)
    net = nets.make_trained_net("LW", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.adam(1e-3, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state, arena = _arena(net, e, 64)
    before = [{k: v.clone() for k, v in b.items()} for b in state.conns]
    for b in state.conns:
        for v in b.values():
            v.zero_()
    arena.write_logical(state.conns)
    for b0, b1 in zip(before, state.conns):
        for k in b0:
            assert torch.equal(b0[k], b1[k]), k


def test_unit_order_agrees_with_the_oracle_restatement(oracle) -> None:
    """The arena's unit renumbering (level, out-degree descending, id) and the
    oracle's independent restatement agree, and hot sources come first in
    their level."""
    e = synth.c2_topological(seed=3, scale=256, layers=5)
    net = nets.make_trained_net("UO", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.sgd(0.1, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state, arena = _arena(net, e, 256)
    conns = [{k: v.numpy().astype(bool) if k == "dead" else v.numpy() for k, v in b.items()}
             for b in state.conns]
    index = oracle.physical_unit_index(state.units["level"].numpy(), conns)
    assert np.array_equal(index, arena.uinv)
    assert np.array_equal(arena.uperm[arena.uinv], np.arange(static.num_units))
    levels = state.units["level"].numpy()[arena.uperm]
    assert (np.diff(levels) >= 0).all()
    deg = np.bincount(e.src, minlength=static.num_units)[arena.uperm]
    for lv in range(levels.max() + 1):
        d = deg[levels == lv]
        assert (np.diff(d) <= 0).all()


def test_units_round_trip_through_the_physical_order() -> None:
    e = synth.c2_topological(seed=7, scale=1024, layers=3)
    net = nets.make_trained_net("UR", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.sgd(0.1, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state, arena = _arena(net, e, 64)
    units = {k: v.clone() for k, v in state.units.items()}
    phys = arena.units_to_physical(units)
    back = arena.units_to_logical(phys)
    for k in units:
        assert torch.equal(units[k], back[k])
    lv = phys["level"].numpy()
    assert (np.diff(lv) >= 0).all()


def test_oracle_and_device_agree_on_the_default_tile(oracle) -> None:
    assert oracle.TILE == _layout.TILE and oracle.NSUPER == _layout.NSUPER


@pytest.mark.parametrize("span,tile,nsuper", [
    (4, 4, 512), (8, 4, 512), (12, 8, 2), (100, 64, 512), (1000, 64, 16), (4096, 4096, 512),
    (4100, 4096, 512), (9590016, 4096, 512), (9590016 + 4, 8192, 512), (123456, 96, 7),
])
def test_tile_partition_agrees_with_the_oracle_restatement(oracle, span, tile, nsuper) -> None:
    """Two independent restatements of the tiling (the layout's tables and
    the oracle's per-position ids) describe the same partition, whose
    superblocks have near-equal length and whose tiles fit the tile size."""
    tile_pos, super_tile = _layout.tile_partition(span, tile, nsuper)
    t_ix, s_ix = oracle.tiles_of_positions(span, tile, nsuper)
    pos = np.arange(span)
    t_of = np.searchsorted(tile_pos, pos, side="right") - 1
    s_of = np.searchsorted(super_tile, t_of, side="right") - 1
    assert np.array_equal(t_of, t_ix) and np.array_equal(s_of, s_ix)
    lens = np.diff(tile_pos)
    assert (lens > 0).all() and (lens <= tile).all() and (tile_pos % 4 == 0).all()
    sb_len = tile_pos[super_tile[1:]] - tile_pos[super_tile[:-1]]
    assert super_tile.size - 1 == min(nsuper, -(-span // tile))
    assert sb_len.max() - sb_len.min() <= 8


def test_one_byte_destinations_fall_back_on_wide_blocks() -> None:
    """A block of 4,096 positions whose live edges span 256 or more
    destination ids keeps the four-byte TO_ID; otherwise every bucket gets
    the one-byte form, exact below live_end."""
    rng = np.random.default_rng(0)
    n_in, n_out = 64, 4096
    src = rng.integers(0, n_in, size=n_out).astype(np.int32)  # one edge per row
    dst = (n_in + np.arange(n_out)).astype(np.int32)
    e = synth.EdgeList(n_in + n_out, src, dst, np.ones(n_out, np.float32), np.arange(n_in, dtype=np.int32),
                       np.arange(n_in, n_in + n_out, dtype=np.int32))
    net = nets.make_trained_net("W", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.sgd(0.1, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    _, _, arena = _arena(net, e, _layout.TILE)
    assert arena.dst8[0] is None
    d8, d0 = _layout.dst_bytes(np.repeat(np.arange(300), 16), 4800)
    assert d8 is not None and d0.tolist() == [0, 256] and int(d8[4096]) == 0 and int(d8[4095]) == 255
    assert _layout.dst_bytes(np.arange(300), 300) == (None, None)


def test_batch_tiles_cover_every_live_edge_once() -> None:
    """The batched update's tiles: every live position once, grouped by 64
    destination x 64 source units (positions ascending inside a group), at
    most BATCH_TILE_EDGES per tile, and loc / tile_base recover each edge's
    ids."""
    rng = np.random.default_rng(3)
    n = 20000
    dst = np.sort(rng.integers(0, 5000, n))
    src = rng.integers(0, 3000, n)
    src[:3000] = 7  # one dense block: a group cut into several tiles
    dst[:3000] = 100
    order = np.lexsort((src, dst))
    src, dst = src[order], dst[order]
    tb = _layout.batch_tiles(src, dst)
    off, base, pos, loc = tb["tile_off"], tb["tile_base"].reshape(-1, 2), tb["pos"], tb["loc"].astype(np.int64)
    assert sorted(pos.tolist()) == list(range(n))
    assert off[0] == 0 and off[-1] == n and (np.diff(off) > 0).all()
    assert (np.diff(off) <= _layout.BATCH_TILE_EDGES).all() and (np.diff(off) == _layout.BATCH_TILE_EDGES).any()
    assert (base % _layout.BATCH_TILE_UNITS == 0).all()
    for k in range(off.size - 1):
        p = pos[off[k] : off[k + 1]]
        assert (np.diff(p) > 0).all()
        assert (base[k, 0] + (loc[off[k] : off[k + 1]] & 0xFF) == dst[p]).all()
        assert (base[k, 1] + (loc[off[k] : off[k + 1]] >> 8) == src[p]).all()


def test_batch_tiles_reject_tables_the_kernel_cannot_take() -> None:
    """batch_tiles validates its own output against the kernel's limits
    (plx_batch_tile_limits); a forged oversize tile is refused."""
    from plastax_amd import _layout

    rng = np.random.default_rng(1)
    src = rng.integers(0, 300, 5000)
    dst = rng.integers(300, 600, 5000)
    tb = _layout.batch_tiles(src, dst)
    assert int(np.diff(tb["tile_off"]).max()) <= _layout.BATCH_TILE_EDGES
    assert int((tb["loc"] & 0xFF).max()) < _layout.BATCH_TILE_UNITS
    # every edge of one (dst block, src block) pair: more than one tile's worth
    many = np.zeros(3 * _layout.BATCH_TILE_EDGES, np.int64)
    tb = _layout.batch_tiles(many, many + 1)
    assert np.diff(tb["tile_off"]).tolist() == [_layout.BATCH_TILE_EDGES] * 3
