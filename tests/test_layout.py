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


def _arena(net, e, tile, **kw):
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cpu", **kw)
    arena = _layout.Arena(static, state.units, state.conns, torch.device("cpu"), tile=tile)
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


def _emulate_fold(arena, b, g_field: np.ndarray):
    """The device's tile fold + partials fold, in numpy float32."""
    bt = arena.bwd[b]
    T = arena.tile
    w = _np(arena.cols["weight"])
    dst = _np(arena.cols["to_id"])
    dead = _np(arena.cols["dead"]).astype(bool)
    sl = _np(bt.sorted_local).view(np.uint16)
    off = _np(bt.grp_off)
    se = _np(bt.grp_se).view(np.uint32)
    tgt = _np(bt.grp_tgt)
    nhot = bt.nhot
    hot = np.zeros(bt.ntiles * nhot, np.float32)
    cold = np.zeros(_np(bt.cold_partial).size, np.float32)
    seen = np.zeros(bt.end - bt.base, np.int64)
    for k in range(bt.ntiles):
        t0 = bt.base + k * T
        n = min(T, bt.end - t0)
        assert off[k] <= off[k + 1]
        for gi in range(off[k], off[k + 1]):
            st, ln = int(se[gi] & 0xFFFF), int(se[gi] >> 16)
            assert ln >= 1 and st + ln <= n
            v = np.float32(0.0)
            for j in range(st, st + ln):
                loc = int(sl[k * T + j])
                assert loc < n
                e = t0 + loc
                assert not dead[e]
                seen[e - bt.base] += 1
                v = np.float32(v + np.float32(w[e] * g_field[dst[e]]))
            if tgt[gi] >= 0:
                cold[tgt[gi]] = v
            else:
                h = -1 - tgt[gi]
                assert 0 <= h < nhot
                hot[k * nhot + h] = v
    live = arena.lives[b]
    assert (seen[:live] == 1).all() and (seen[live:] == 0).all()
    rows = _np(bt.rows)
    row_hot = _np(bt.row_hot)
    row_cold = _np(bt.row_cold)
    assert row_cold[0] == 0 and (np.diff(row_cold) >= 0).all() and row_cold[-1] == cold.size or (cold.size == 1 and row_cold[-1] == 0)
    cold_sb = _np(bt.cold_sb).view(np.uint16)
    SB = _layout.SUPERBLOCK
    out = {}
    for r in range(rows.size):
        s = np.float32(0.0)
        if row_hot[r] >= 0:
            for k0 in range(0, bt.ntiles, SB):
                q = np.float32(0.0)
                for k in range(k0, min(k0 + SB, bt.ntiles)):
                    q = np.float32(q + hot[k * nhot + row_hot[r]])
                s = np.float32(s + q)
        else:
            j0, j1 = row_cold[r], row_cold[r + 1]
            if j0 < j1:
                cur, q = cold_sb[j0], np.float32(0.0)
                for j in range(j0, j1):
                    if cold_sb[j] != cur:
                        s, q, cur = np.float32(s + q), np.float32(0.0), cold_sb[j]
                    q = np.float32(q + cold[j])
                s = np.float32(s + q)
        out[int(rows[r])] = s
    return out


@pytest.mark.parametrize("tile", [64, 256])
def test_tiled_fold_emulation_matches_oracle_exactly(oracle, tile: int) -> None:
    e = synth.c2_topological(seed=2, scale=512, layers=4)
    net = nets.make_trained_net("L", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.sgd(0.1, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state, arena = _arena(net, e, tile)
    _check_arena(static, state, arena)
    o = nets.oracle_for(oracle, net, static, state, tile=tile)
    rng = np.random.default_rng(0)
    g = rng.standard_normal(static.num_units).astype(np.float32)
    o.units["grad_pre_act"][:] = g
    assert any(arena.bwd[b].nhot > 0 for b in range(1, arena.num_buckets))
    for b in range(1, arena.num_buckets):
        got = _emulate_fold(arena, b, g)
        want = o._reduce_bwd(b, "grad_pre_act", 0)
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
    want = o._reduce_bwd(0, "grad_pre_act", 0)
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


def test_oracle_and_device_agree_on_the_default_tile(oracle) -> None:
    assert oracle.TILE == _layout.TILE
