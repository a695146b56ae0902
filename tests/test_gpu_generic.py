"""Generic passes on the device (plastax_amd/generic.py, plx_gen_fold):
bit-exact with the oracle's generic path over training steps.

Cases: a nonlinear forward map with the product backward (tiled layout);
a tuple forward accumulator under (sum, max, sum) with a three-factor
backward map (both generic: the churn layout's source lists), TOPOLOGICAL
and PIPELINE; and a product map written as a one-element tuple, whose device
run must equal the product kernels' bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import generic_cases as gc
import nets
import plastax_amd as px
from test_gpu_parity import _equal, assert_same_state

pytestmark = pytest.mark.gpu


def _run(oracle, net, pipeline: bool, steps: int, seed: int, arena_mode: str = "auto"):
    static, state = gc.build(net, pipeline=pipeline, seed=seed, device="cuda")
    o = nets.oracle_for(oracle, net, static, state)
    step = px.make_step(net, static)
    step.arena_mode = arena_mode
    if step.backward_order == "slot":
        o.tile = None
    xs, ts = gc.data(seed + 1, steps, len(static.input_ids), len(static.output_ids))
    losses = []
    for k in range(steps):
        print(f"generic step {k} {net.forward_pass.__class__.__name__} pipeline={pipeline}", flush=True)
        res = step(state, px.StepInputs(xs[k], ts[k]))
        state = res.state
        lo = o.step(xs[k], ts[k])
        torch.cuda.synchronize()
        assert_same_state(static, state, o, f"step {k}")
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at step {k}"
        losses.append(float(res.loss))
    return static, state, losses


@pytest.mark.parametrize(
    ("forward", "backward", "pipeline"),
    [
        (gc.TanhSrcForward(), nets.TanhBackward(), False),
        (gc.TupleForward(), gc.ThreeFactorBackward(), False),
        (gc.TupleForward(), gc.ThreeFactorBackward(), True),
    ],
)
def test_generic_passes_match_the_oracle(oracle, forward, backward, pipeline: bool) -> None:
    net = gc.make_net(forward, backward, pipeline=pipeline, optimizer=px.optim.adam(1e-2, nets.GRAD_PRE_ACT))
    _run(oracle, net, pipeline, 6, 11)


def test_generic_backward_on_the_tiled_layout(oracle) -> None:
    """arena_mode="tiled": the generic backward folds each source's
    out-edges in slot order from the tiled arena's batch_sources lists."""
    net = gc.make_net(gc.TupleForward(), gc.ThreeFactorBackward(), optimizer=px.optim.adam(1e-2, nets.GRAD_PRE_ACT))
    _run(oracle, net, False, 5, 13, arena_mode="tiled")


def test_product_map_as_a_tuple_matches_the_product_kernels(oracle) -> None:
    prod = gc.make_net(nets.TanhForward(), nets.TanhBackward())
    gen = gc.make_net(gc.ProductAsTupleForward(), gc.ProductAsTupleBackward())
    sp, st_p = gc.build(prod, pipeline=False, seed=5, device="cuda")
    step_p = px.make_step(prod, sp)
    step_p.arena_mode = "churn"  # the generic backward's slot order
    xs, ts = gc.data(6, 5, len(sp.input_ids), len(sp.output_ids))
    for k in range(5):
        st_p = step_p(st_p, px.StepInputs(xs[k], ts[k])).state
    _, st_g, _ = _run(oracle, gen, False, 5, 5)
    hp, hg = nets.host_units(sp, st_p), nets.host_units(sp, st_g)
    for name in hp:
        assert np.array_equal(hp[name].view(np.uint8), hg[name].view(np.uint8)), name
    for a, b in zip(nets.host_conns(sp, st_p), nets.host_conns(sp, st_g)):
        for name in a:
            assert np.array_equal(np.asarray(a[name]).view(np.uint8), np.asarray(b[name]).view(np.uint8)), name


@pytest.mark.parametrize(
    ("forward", "backward", "B"),
    [
        (gc.TanhSrcForward(), nets.TanhBackward(), 3),
        (gc.TupleForward(), gc.ThreeFactorBackward(), 4),
        (gc.TupleForward(), gc.ThreeFactorBackward(), 1),
    ],
)
def test_batched_generic_passes_match_the_batched_oracle(oracle, forward, backward, B: int) -> None:
    """A generic forward / backward per sample (step.py:443-447): the fold
    per (row, sample), the apply per (finalized unit, sample), the apply's
    written columns batch-reduced (phases.py:298-387) -- against the batched
    oracle bit for bit."""
    from oracle import batched as ob

    base = gc.make_net(forward, backward, optimizer=px.optim.adam(1e-2, nets.GRAD_PRE_ACT))

    class Batched(base):
        batch_reduction = px.MeanFloatFirstRest()

    static, state = gc.build(Batched, pipeline=False, seed=7, device="cuda")
    o = nets.oracle_for(oracle, Batched, static, state)
    orc = ob.OracleBatch(o, B)
    step = px.make_step(Batched, static, batch_size=B)
    rng = np.random.default_rng(8)
    n_in, n_out = len(static.input_ids), len(static.output_ids)
    for k in range(4):
        x = rng.standard_normal((B, n_in)).astype(np.float32)
        t = rng.standard_normal((B, n_out)).astype(np.float32)
        print(f"batched generic pass step {k} B={B} {forward.__class__.__name__}", flush=True)
        res = step(state, px.StepInputs(x, t))
        state = res.state
        lo = orc.step(x, t)
        torch.cuda.synchronize()
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at step {k}"
        assert_same_state(static, state, o, f"step {k}")


class _TauPrune(px.PruneConn):
    def predicate(self, u, c, cid, g):
        return px.numpy.abs(c[px.WEIGHT, cid]) < np.float32(0.03)


class _Grow(px.ScoreAddConn):
    candidates = "shortlist_per_level"
    shortlist_size = 8
    direction = "deeper"
    dedupe_live = True
    max_new_per_level = 10

    def score(self, u, src, dst, g):
        return px.numpy.abs(u[px.ACTIVATION, src] * u[nets.GRAD_PRE_ACT, dst])

    def importance(self, u, i, g):
        return px.numpy.abs(u[nets.GRAD_PRE_ACT, i]) + px.numpy.abs(u[px.ACTIVATION, i])

    def init(self, u, src, dst, g):
        return px.ConnWrite.of((px.WEIGHT, np.float32(0.0)))


@pytest.mark.parametrize("B", [None, 3])
def test_generic_passes_with_pruning_and_growth(oracle, B) -> None:
    """Tombstones inside the backward's per-source lists (PruneConn each
    step) and a new layout after every growth, under a generic forward and
    backward: the streaming step on the tiled layout (B None) and a batched
    step (B = 3), against the oracle bit for bit."""
    from oracle import batched as ob

    base = gc.make_net(gc.TupleForward(), gc.ThreeFactorBackward(), optimizer=px.optim.adam(1e-2, nets.GRAD_PRE_ACT))

    class Net(base):
        prune_conn = _TauPrune()
        add_conn = _Grow()
        batch_reduction = px.MeanFloatFirstRest()

    static, state = gc.build(Net, pipeline=False, seed=7, device="cuda")
    o = nets.oracle_for(oracle, Net, static, state)
    if B is None:
        step = px.make_step(Net, static)
        step.arena_mode = "tiled"
    else:
        step = px.make_step(Net, static, batch_size=B)
        orc = ob.OracleBatch(o, B)
    rng = np.random.default_rng(8)
    n_in, n_out = len(static.input_ids), len(static.output_ids)
    for k in range(4):
        nb = B or 1
        x = rng.standard_normal((nb, n_in)).astype(np.float32)
        t = rng.standard_normal((nb, n_out)).astype(np.float32)
        print(f"generic prune+growth step {k} B={B}", flush=True)
        if B is None:
            res = step(state, px.StepInputs(x[0], t[0]))
            lo = o.step(x[0], t[0])
        else:
            res = step(state, px.StepInputs(x, t))
            lo = orc.step(x, t)
        state = res.state
        torch.cuda.synchronize()
        assert (state.grown, state.overflow) == (o.grown, o.overflow), f"flags at step {k}"
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at step {k}"
        assert_same_state(static, state, o, f"step {k}")
    assert o.grown > 0 and sum(int(c["dead"].sum()) for c in o.conns) > 0
