"""Generic passes (maps outside the product form, tuple accumulators) in the
plan and in the oracle, on the host.

The oracle's generic path is pinned two ways: a product map written as a
one-element tuple runs through it and must give the product path's bits
(same fold order: each row's live edges in slot order); and a tuple
accumulator's components must equal their closed forms: the count
component the in-degree, the max component (written to its own column) the
numpy scatter-max of |w| * util over each destination's live in-edges,
-inf where a row has none. The min and prod components are pinned the same
way in test_monoid_oracle.py.
"""

from __future__ import annotations

import numpy as np
import pytest

import generic_cases as gc
import nets
import plastax_amd as px
from plastax_amd._plan import compile_plan


def _oracle(oracle, net, static, state):
    o = nets.oracle_for(oracle, net, static, state)
    o.tile = None  # each source's backward terms in slot order
    return o


@pytest.mark.parametrize("pipeline", [False, True])
def test_generic_oracle_gives_the_product_paths_bits(oracle, pipeline: bool) -> None:
    prod = gc.make_net(nets.TanhForward(), nets.TanhBackward(), pipeline=pipeline)
    gen = gc.make_net(gc.ProductAsTupleForward(), gc.ProductAsTupleBackward(), pipeline=pipeline)
    assert compile_plan(gen, gc.build(gen, pipeline=pipeline, seed=1)[0]).forward.generic is not None
    runs = []
    for net in (prod, gen):
        static, state = gc.build(net, pipeline=pipeline, seed=1)
        o = _oracle(oracle, net, static, state)
        xs, ts = gc.data(2, 5, len(static.input_ids), len(static.output_ids))
        losses = [o.step(xs[k], ts[k]) for k in range(5)]
        runs.append((losses, o.units, o.conns))
    (la, ua, ca), (lb, ub, cb) = runs
    assert np.array_equal(np.float32(la).view(np.uint32), np.float32(lb).view(np.uint32))
    for name in ua:
        assert np.array_equal(np.asarray(ua[name]).view(np.uint8), np.asarray(ub[name]).view(np.uint8)), name
    for a, b in zip(ca, cb):
        for name in a:
            assert np.array_equal(np.asarray(a[name]).view(np.uint8), np.asarray(b[name]).view(np.uint8)), name


def test_tuple_accumulator_components_match_closed_forms(oracle) -> None:
    net = gc.make_net(gc.TupleForward(), nets.TanhBackward())
    static, state = gc.build(net, pipeline=False, seed=3)
    o = _oracle(oracle, net, static, state)
    rng = np.random.default_rng(0)
    for c in o.conns:  # a varied UTIL column
        c[gc.UTIL.name] = rng.random(c["dead"].size).astype(np.float32)
        live = np.flatnonzero(c["dead"] == 0)
        c["dead"][live[::9]] = 1  # tombstones inside the rows
        c["dead"][c["to_id"] == 30] = 1  # a level-1 row with no live in-edge
    x = rng.standard_normal(len(static.input_ids)).astype(np.float32)
    o.units["activation"][np.asarray(static.input_ids)] = x
    o.forward()
    n = static.num_units
    deg = np.zeros(n, np.int64)
    mx = np.full(n, -np.inf, np.float32)
    for c in o.conns:
        live = ~c["dead"].astype(bool)
        np.add.at(deg, c["to_id"][live], 1)
        np.maximum.at(mx, c["to_id"][live], np.abs(c["weight"][live]) * c[gc.UTIL.name][live])
    is_in = np.zeros(n, bool)
    is_in[np.asarray(static.input_ids)] = True
    fin = ~is_in & (o.units["level"] >= 1)
    assert np.array_equal(o.units[gc.DEG.name][fin], deg[fin].astype(np.float32))
    got = o.units[gc.MX.name][fin]
    assert np.array_equal(got.view(np.uint32), mx[fin].view(np.uint32))
    assert deg[30] == 0 and o.units[gc.MX.name][30] == -np.inf
    assert np.array_equal(np.isneginf(got), deg[fin] == 0)


def test_plan_marks_generic_passes_and_batched_steps_reduce_their_writes() -> None:
    net = gc.make_net(gc.TanhSrcForward(), nets.TanhBackward())
    static, _ = gc.build(net, pipeline=False, seed=4)
    plan = compile_plan(net, static)
    assert plan.forward.generic is not None and plan.backward.generic is None
    assert plan.forward.generic.why  # the product form's refusal, kept for the record
    tup = gc.make_net(gc.TupleForward(), gc.ThreeFactorBackward())
    static2, _ = gc.build(tup, pipeline=False, seed=4)
    plan2 = compile_plan(tup, static2)
    assert plan2.forward.generic.tuple_acc and plan2.forward.generic.monoids == (0, 2, 0)
    assert plan2.backward.generic is not None and not plan2.backward.generic.tuple_acc

    class Batched(tup):
        batch_reduction = px.MeanFloatFirstRest()

    bstep = px.make_step(Batched, static2, batch_size=4)
    assert not bstep.churn()  # the batched backward reads batch_sources' lists on the tiled layout
    red = bstep._check_policy(gc.build(Batched, pipeline=False, seed=4)[1].globals_)
    # the generic applies' writes are batch-reduced: ACTIVATION and DEG
    # (forward), GRAD_PRE_ACT (backward), with MeanFloatFirstRest's MEAN
    assert red[gc.DEG.name] is px.Reduction.MEAN and red[nets.GRAD_PRE_ACT.name] is px.Reduction.MEAN
    step = px.make_step(tup, static2)
    assert step.churn()  # a generic backward folds each source's out-edges from the churn lists
    step.arena_mode = "tiled"
    assert not step.churn()  # a tiled arena's generic backward reads batch_sources' lists


@pytest.mark.parametrize("B", [1, 3])
def test_batched_generic_oracle_gives_the_product_paths_bits(oracle, B: int) -> None:
    """The batched oracle on a generic net whose maps have the product form
    gives the batched product path's bits (every unit column, every
    connection column, the loss), so the batched generic writes are reduced
    exactly as the product outputs are; at B = 1 both are the streaming step
    (tests/test_batched.py:117-140)."""
    from oracle import batched as ob

    runs = []
    for fwd, bwd in ((nets.TanhForward(), nets.TanhBackward()),
                     (gc.ProductAsTupleForward(), gc.ProductAsTupleBackward())):
        base = gc.make_net(fwd, bwd)

        class Batched(base):
            batch_reduction = px.MeanFloatFirstRest()

        static, state = gc.build(Batched, pipeline=False, seed=2)
        orc = ob.OracleBatch(_oracle(oracle, Batched, static, state), B)
        rng = np.random.default_rng(3)
        n_in, n_out = len(static.input_ids), len(static.output_ids)
        losses = []
        for _ in range(3):
            x = rng.standard_normal((B, n_in)).astype(np.float32)
            t = rng.standard_normal((B, n_out)).astype(np.float32)
            losses.append(orc.step(x, t))
        runs.append((losses, orc.o.units, orc.o.conns))
    if B == 1:  # and the streaming oracle on the same inputs
        static, state = gc.build(gc.make_net(nets.TanhForward(), nets.TanhBackward()), pipeline=False, seed=2)
        o = _oracle(oracle, gc.make_net(nets.TanhForward(), nets.TanhBackward()), static, state)
        rng = np.random.default_rng(3)
        losses = []
        for _ in range(3):
            x = rng.standard_normal((1, len(static.input_ids))).astype(np.float32)
            t = rng.standard_normal((1, len(static.output_ids))).astype(np.float32)
            losses.append(o.step(x[0], t[0]))
        runs.append((losses, o.units, o.conns))
    (la, ua, ca) = runs[0]
    for lb, ub, cb in runs[1:]:
        assert np.array_equal(np.float32(la).view(np.uint32), np.float32(lb).view(np.uint32))
        for name in ua:
            assert np.array_equal(np.asarray(ua[name]).view(np.uint8), np.asarray(ub[name]).view(np.uint8)), name
        for a, b in zip(ca, cb):
            for name in a:
                assert np.array_equal(np.asarray(a[name]).view(np.uint8), np.asarray(b[name]).view(np.uint8)), name
