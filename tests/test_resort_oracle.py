"""The CPU restatement of topo.resort and grow_bucket (topo.py:189-452,
state.py:238-313), pinned by what fixes it independently:

- the relaxed levels equal the builder's longest-path levels
  (plastax_amd.topo.initial_levels, the frontier Kahn walk of topo.py:35-130)
  on random DAGs whose in-degree-0 units are the inputs;
- every live edge lands in the bucket of its source's new level, the buckets
  are sorted stably by source (old relative order within a source), dead
  edges are dropped, and capacities never shrink;
- a cycle raises in TOPOLOGICAL mode; PIPELINE keeps one bucket and resets
  the tail to the live count;
- grow_bucket pads with never-used slots to max(policy(live + 1), 2 x old).
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest

import plastax_amd as px
from nets import ReluForward
from oracle import growth as og
from plastax_amd import topo
from plastax_amd.state import column_to_numpy


def _net(pipeline: bool = False):
    class Net(px.Network):
        forward_pass = ReluForward()
        propagation = px.Propagation.PIPELINE if pipeline else px.Propagation.TOPOLOGICAL

    return Net


def _build(n, src, dst, inputs, pipeline=False, headroom=0.5):
    net = _net(pipeline)
    static, state = px.NetworkBuilder.from_edges(
        net, n, np.asarray(src, np.int32), np.asarray(dst, np.int32),
        weights=np.arange(len(src), dtype=np.float32), input_ids=list(inputs), output_ids=[n - 1],
        globals_=None, capacity_headroom=headroom, device="cpu")
    us = {s.name: s for s in static.unit_fields}
    cs = {s.name: s for s in static.conn_fields}
    units = {k: column_to_numpy(v, us[k]).copy() for k, v in state.units.items()}
    conns = [{k: column_to_numpy(v, cs[k]).copy() for k, v in b.items()} for b in state.conns]
    return static, units, conns


def _random_dag(rng, n, m, n_in):
    order = rng.permutation(n - n_in) + n_in
    pos = np.empty(n, np.int64)
    pos[:n_in] = -1
    pos[order] = np.arange(n - n_in)
    src = rng.integers(0, n, m)
    dst = rng.integers(n_in, n, m)
    keep = pos[src] < pos[dst]
    src, dst = src[keep], dst[keep]
    # every non-input unit gets an incoming edge from an input (in-degree 0 = inputs)
    src = np.concatenate([src, rng.integers(0, n_in, n - n_in)])
    dst = np.concatenate([dst, np.arange(n_in, n)])
    return src, dst


@pytest.mark.parametrize("seed", range(4))
def test_relaxed_levels_equal_the_builders_longest_path(seed: int) -> None:
    rng = np.random.default_rng(seed)
    n, n_in = 300, 6
    src, dst = _random_dag(rng, n, 900, n_in)
    static, units, conns = _build(n, src, dst, range(n_in))
    lv, converged = og.relax_levels(static, conns, pin_inputs=True, rounds=n)
    assert converged
    want = topo.initial_levels(n, np.stack([src, dst], 1), input_ids=tuple(range(n_in)))
    assert np.array_equal(lv, want)


def test_resort_regroups_by_new_level() -> None:
    rng = np.random.default_rng(9)
    n, n_in = 200, 5
    src, dst = _random_dag(rng, n, 600, n_in)
    static, units, conns = _build(n, src, dst, range(n_in))
    # kill some edges and add a deeper edge into a shallow bucket's free slot
    flat_dead = [c["dead"].copy() for c in conns]
    for c in conns:
        live = np.flatnonzero(~c["dead"].astype(bool))
        c["dead"][live[::7]] = True
    b0 = conns[0]
    free = np.flatnonzero(b0["dead"].astype(bool))[0]
    deep = int(np.argmax(units["level"]))
    b0["from_id"][free], b0["to_id"][free], b0["dead"][free] = 0, deep, False
    new_static, new_units, new_conns, tail = og.resort(static, units, conns)
    lv = new_units["level"]
    flat = {k: np.concatenate([c[k] for c in conns]) for k in conns[0]}
    live = ~flat["dead"].astype(bool)
    assert tail == 0
    total = 0
    for b, c in enumerate(new_conns):
        d = c["dead"].astype(bool)
        k = int((~d).sum())
        assert not d[:k].any() and d[k:].all()
        assert (lv[c["from_id"][:k]] == b).all()
        assert (np.diff(c["from_id"][:k]) >= 0).all()
        # within one source, the old relative (flat) order: weights are the
        # original edge indices and were laid out source-major by the builder
        assert c["dead"].shape[0] >= (static.level_capacities[b] if b < len(static.level_capacities) else 0)
        total += k
    assert total == int(live.sum())
    assert len(new_conns) == int(lv.max())
    del flat_dead


def test_resort_rejects_a_cycle_and_pipeline_keeps_one_bucket() -> None:
    static, units, conns = _build(4, [0, 1, 2], [1, 2, 3], [0])
    b = conns[1]
    free = np.flatnonzero(b["dead"].astype(bool))[0]
    b["from_id"][free], b["to_id"][free], b["dead"][free] = 2, 1, False  # 1 -> 2 -> 1
    with pytest.raises(ValueError, match="cycle"):
        og.resort(static, units, conns)
    ps, pu, pc = _build(4, [0, 1, 2, 2], [1, 2, 1, 3], [0], pipeline=True)
    pc[0]["dead"][1] = True
    s2, u2, c2, tail = og.resort(ps, pu, pc)
    assert len(c2) == 1 and tail == 3
    assert s2.level_capacities[0] >= ps.level_capacities[0]


def test_grow_bucket_pads_with_never_used_slots() -> None:
    static, units, conns = _build(6, [0, 0, 1, 2, 3], [2, 3, 4, 5, 5], [0, 1], headroom=0.0)
    old = static.level_capacities
    s2, c2 = og.grow_bucket(static, conns, 1)
    assert s2.level_capacities[1] == max(topo.capacity_policy(int((~conns[1]["dead"].astype(bool)).sum()) + 1),
                                         2 * old[1])
    assert (c2[1]["dead"][old[1]:]).all()
    for name in conns[1]:
        assert np.array_equal(c2[1][name][: old[1]], conns[1][name])
    aligned = dataclasses.replace(static, capacity_align=8)
    s3, _ = og.grow_bucket(aligned, conns, 0)
    assert s3.level_capacities[0] == max(topo.capacity_policy(int((~conns[0]["dead"].astype(bool)).sum()) + 1,
                                                              align=8),
                                         topo.capacity_policy(old[0] + old[0] // 2, align=8))
