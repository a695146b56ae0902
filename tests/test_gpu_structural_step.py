"""Streaming steps with structural phases: device vs oracle, bit for bit.

Training steps (forward, loss, backward, Adam / SGD update) followed by
PruneConn and add_conn, as the reference's phase order runs them
(phases.py:87-182), over many steps: tombstones set in place on the device's
laid-out arena, growth on the logical arena, the layout rebuilt after each
growth. The oracle runs the same phases on host arrays; units, every logical
connection column and the loss must agree bit for bit at the checked steps,
and the structural flags at every step.

- a C4-shaped dynamic sparse MLP (scaled down): PruneConn |w| < g["tau"]
  with tau raised every 5 steps, regrowth by a per-level shortlist scored
  by |act * grad| with direction "deeper" and dedupe_live;
- a C5-shaped growing reservoir (scaled down): PIPELINE, per-unit
  proposals (P = 4) every step, pruning of small weights.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import nets
import plastax_amd as px
import plastax_amd.numpy as jnp
from test_gpu_parity import _equal, assert_same_state

pytestmark = pytest.mark.gpu


class TauPrune(px.PruneConn):
    def predicate(self, u, c, cid, g):
        return jnp.abs(c[px.WEIGHT, cid]) < g["tau"]


class GradGrow(px.ScoreAddConn):
    candidates = "shortlist_per_level"
    shortlist_size = 24
    direction = "deeper"
    dedupe_live = True
    max_new_per_level = 40
    trigger = ("every", 5)

    def score(self, u, src, dst, g):
        return jnp.abs(u[px.ACTIVATION, src] * u[nets.GRAD_PRE_ACT, dst])

    def importance(self, u, i, g):
        return jnp.abs(u[nets.GRAD_PRE_ACT, i]) + jnp.abs(u[px.ACTIVATION, i]) * jnp.float32(0.25)

    def init(self, u, src, dst, g):
        return px.ConnWrite.of((px.WEIGHT, jnp.float32(0.0)))


def _sparse_mlp(rng: np.random.Generator, layers: list[int], keep: float):
    src, dst = [], []
    base = np.concatenate([[0], np.cumsum(layers)])
    for l in range(len(layers) - 1):
        a = np.arange(base[l], base[l + 1])
        b = np.arange(base[l + 1], base[l + 2])
        m = rng.random((a.size, b.size)) < keep
        ii, jj = np.nonzero(m)
        src.append(a[ii])
        dst.append(b[jj])
    src = np.concatenate(src).astype(np.int32)
    dst = np.concatenate(dst).astype(np.int32)
    fan = np.bincount(dst, minlength=int(base[-1]))
    w = (rng.standard_normal(src.size) / np.sqrt(np.maximum(fan[dst], 1))).astype(np.float32)
    return int(base[-1]), src, dst, w, np.arange(layers[0]), np.arange(base[-2], base[-1])


def _run(net, static, state, oracle, inputs_fn, globals_fn, steps, check_at):
    o = nets.oracle_for(oracle, net, static, state)
    o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
    step = px.make_step(net, static)
    if step.backward_order == "slot":
        o.tile = None  # the churn layout folds each source's edges in slot order
    grown_total = 0
    for k in range(1, steps + 1):
        g = globals_fn(k)
        state.globals_ = g
        o.globals_ = g
        x, t = inputs_fn(k)
        print(f"structural step {k}", flush=True)
        res = step(state, px.StepInputs(x, t))
        state = res.state
        lo = o.step(x, t)
        assert (state.grown, state.overflow, state.needs_resort, state.tail_start) == (
            o.grown, o.overflow, o.needs_resort, o.tail_start), f"flags at step {k}"
        grown_total += state.grown
        if k in check_at:
            torch.cuda.synchronize()
            assert_same_state(static, state, o, f"step {k}")
            assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at {k}"
    return state, o, grown_total


def test_dynamic_sparse_mlp_prune_and_regrow_bit_exact(oracle) -> None:
    rng = np.random.default_rng(4)
    n, src, dst, w, ins, outs = _sparse_mlp(rng, [96, 256, 256, 10], 0.1)
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT)

    class DST(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        prune_conn = TauPrune()
        add_conn = GradGrow()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        extra_conn_fields = tuple(opt.state_fields)

    static, state = px.NetworkBuilder.from_edges(
        DST, n, src, dst, weights=w, input_ids=ins, output_ids=outs,
        globals_={"tau": np.float32(0.0)}, capacity_headroom=0.25, device="cuda")
    teacher = rng.standard_normal((10, 96)).astype(np.float32) * np.float32(0.1)
    xs = rng.random((30, 96)).astype(np.float32)

    def inputs(k):
        x = xs[k - 1]
        return x, np.tanh(teacher @ x).astype(np.float32)

    def globals_fn(k):
        # Prune before every growth (steps 1, 6, 11, 16) and on its own in
        # between (steps 3, 8, 13: tombstones inside the laid-out arena).
        tau = 0.02 if (k - 1) % 5 == 0 else (0.005 if k % 5 == 3 else 0.0)
        return {"tau": np.float32(tau)}

    _, o, grown = _run(DST, static, state, oracle, inputs, globals_fn, 16, {1, 2, 3, 4, 5, 6, 9, 11, 16})
    assert grown > 0


class Propose4(px.ProposeAddConn):
    proposer = "per_unit"
    proposals_per_proposer = 4
    max_new_per_level = 6
    max_level_gap = 1 << 20

    def propose(self, u, i, j, g, rng):
        dst = rng.uniform_int(2048).astype(jnp.int32)
        return jnp.asarray(i, jnp.int32), dst, rng.uniform() + jnp.abs(u[px.ACTIVATION, i])

    def init(self, u, src, dst, g):
        return px.ConnWrite.of((px.WEIGHT, jnp.float32(0.05)))


def test_growing_reservoir_propose_and_prune_bit_exact(oracle) -> None:
    rng = np.random.default_rng(5)
    n, m = 2048, 16384
    src = rng.integers(0, n, m).astype(np.int32)
    dst = rng.integers(0, n, m).astype(np.int32)
    keep = src != dst
    src, dst = src[keep], dst[keep]
    w = (rng.standard_normal(src.size) * 0.25).astype(np.float32)
    opt = px.optim.sgd(1e-2, nets.GRAD_PRE_ACT)

    class Reservoir(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        prune_conn = TauPrune()
        add_conn = Propose4()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        propagation = px.Propagation.PIPELINE

    static, state = px.NetworkBuilder.from_edges(
        Reservoir, n, src, dst, weights=w, input_ids=np.arange(64), output_ids=np.arange(n - 16, n),
        globals_={"tau": np.float32(0.0)}, capacity_headroom=1.0, device="cuda")
    xs = rng.standard_normal((20, 64)).astype(np.float32)

    def inputs(k):
        x = xs[k - 1]
        return x, np.tanh(x[:16]).astype(np.float32)

    def globals_fn(k):
        return {"tau": np.float32(0.01 * (k % 3))}

    _, o, grown = _run(Reservoir, static, state, oracle, inputs, globals_fn, 12, {1, 3, 7, 12})
    assert grown > 0


TRACE = px.FieldSpec.float32("trace", 0.5)


class DecayTrace(px.UpdateUnit):
    def update(self, u, i, g):
        return px.UnitWrite.of((TRACE, u[TRACE, i] * jnp.float32(0.75) + jnp.abs(u[px.ACTIVATION, i])))


class PruneSaturated(px.PruneUnit):
    def predicate(self, u, i, g):
        return u[TRACE, i] > g["trace_max"]


class SpawnCold(px.AddUnit):
    def spawn(self, u, parent, g):
        return u[TRACE, parent] < g["trace_min"], jnp.int32(1)

    def init(self, u, child, parent, g):
        return px.UnitWrite.of((px.ACTIVATION, u[px.ACTIVATION, parent] * jnp.float32(0.5)),
                               (TRACE, jnp.float32(0.25)))


@pytest.mark.parametrize("pipeline", [True, False])
def test_full_churn_bit_exact(oracle, pipeline: bool) -> None:
    """update_unit between the backward and the update, prune_unit with its
    incident-edge kill, add_unit every 3rd step, PruneConn and growth:
    device vs oracle every step."""
    rng = np.random.default_rng(6 + pipeline)
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT)
    if pipeline:
        n_alloc, cap = 1500, 2048
        src = rng.integers(0, n_alloc, 9000).astype(np.int32)
        dst = rng.integers(0, n_alloc, 9000).astype(np.int32)
        keep = src != dst
        src, dst = src[keep], dst[keep]
        w = (rng.standard_normal(src.size) * 0.3).astype(np.float32)
        ins, outs = np.arange(32), np.arange(n_alloc - 8, n_alloc)
        grow_rule = Propose4()
    else:
        n_alloc, src, dst, w, ins, outs = _sparse_mlp(rng, [64, 200, 200, 10], 0.15)
        cap = n_alloc + 200
        grow_rule = GradGrow()

    class Churn(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        update_unit = DecayTrace()
        prune_unit = PruneSaturated()
        prune_conn = TauPrune()
        add_unit = SpawnCold()
        add_conn = grow_rule
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD, TRACE)
        extra_conn_fields = tuple(opt.state_fields)
        unit_capacity = cap
        structural_interval = 3
        propagation = px.Propagation.PIPELINE if pipeline else px.Propagation.TOPOLOGICAL

    g0 = {"tau": np.float32(0.0), "trace_max": np.float32(2.6), "trace_min": np.float32(0.3 if pipeline else 0.7)}
    static, state = px.NetworkBuilder.from_edges(
        Churn, n_alloc, src, dst, weights=w, input_ids=ins, output_ids=outs, globals_=g0,
        capacity_headroom=1.0, device="cuda")
    n_in, n_out = len(ins), len(outs)
    teacher = rng.standard_normal((n_out, n_in)).astype(np.float32) * np.float32(0.3)
    xs = rng.standard_normal((14, n_in)).astype(np.float32)

    def inputs(k):
        x = xs[k - 1]
        return x, np.tanh(teacher @ x).astype(np.float32)

    def globals_fn(k):
        return {**g0, "tau": np.float32(0.004 * (k % 2))}

    o = nets.oracle_for(oracle, Churn, static, state)
    o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
    step = px.make_step(Churn, static)
    if step.backward_order == "slot":
        o.tile = None
    added = 0
    for k in range(1, 13):
        g = globals_fn(k)
        state.globals_ = g
        o.globals_ = g
        x, t = inputs(k)
        print(f"churn step {k} pipeline={pipeline}", flush=True)
        res = step(state, px.StepInputs(x, t))
        state = res.state
        lo = o.step(x, t)
        assert (state.units_added, state.unit_overflow, state.grown, state.overflow, state.tail_start) == (
            o.units_added, o.unit_overflow, o.grown, o.overflow, o.tail_start), f"flags at step {k}"
        added += state.units_added
        torch.cuda.synchronize()
        assert_same_state(static, state, o, f"step {k}")
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at {k}"
    assert added > 0


class SetProposeGrow(px.ProposeAddConn):
    """The proposer of examples/dst_sparse.py:296-337 (SET with proposals):
    each unit proposes P edges into a random unit of the next layer with a
    random priority, read from constant layer tables at the traced layer
    index, and returns a px.Proposal."""

    proposer = "per_unit"

    def __init__(self, max_new_per_level, grow_scale, layer_sizes, proposals_per_unit=16):
        self.max_new_per_level = max_new_per_level
        self.proposals_per_proposer = proposals_per_unit
        self.direction = "deeper"
        self.dedupe_live = True
        self.dedupe_step = True
        self.grow_scale = grow_scale
        sizes = np.asarray(layer_sizes, dtype=np.int32)
        starts = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
        self._next_start = jnp.asarray(starts[1:])
        self._next_width = jnp.asarray(np.append(sizes[1:], 0).astype(np.int32))

    def propose(self, u, i, j, g, rng):
        layer = jnp.sum(i >= self._next_start)
        width = self._next_width[layer]
        offset = (rng.uniform() * width.astype(jnp.float32)).astype(jnp.int32)
        dst = self._next_start[layer] + jnp.minimum(offset, width - 1)
        score = jnp.where(width > 0, rng.uniform(), -jnp.inf)
        return px.Proposal(src=i, dst=dst, score=score)

    def init(self, u, src, dst, g):
        return px.ConnWrite.of((px.WEIGHT, jnp.float32(self.grow_scale)))


def test_set_proposer_returning_proposals_bit_exact(oracle) -> None:
    """A sparse MLP pruned by |w| < tau and regrown every step by the SET
    proposer (P = 4, 24 per level, live and step dedupe): flags every step,
    every column at the checked steps, bit for bit with the oracle."""
    rng = np.random.default_rng(6)
    layers = [96, 256, 256, 10]
    n, src, dst, w, ins, outs = _sparse_mlp(rng, layers, 0.1)
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT)

    class SET(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        prune_conn = TauPrune()
        add_conn = SetProposeGrow(24, 0.01, tuple(layers), proposals_per_unit=4)
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        extra_conn_fields = tuple(opt.state_fields)

    static, state = px.NetworkBuilder.from_edges(
        SET, n, src, dst, weights=w, input_ids=ins, output_ids=outs,
        globals_={"tau": np.float32(0.0)}, capacity_headroom=0.25, device="cuda")
    teacher = rng.standard_normal((10, 96)).astype(np.float32) * np.float32(0.1)
    xs = rng.random((12, 96)).astype(np.float32)

    def inputs(k):
        x = xs[k - 1]
        return x, np.tanh(teacher @ x).astype(np.float32)

    def globals_fn(k):
        return {"tau": np.float32(0.01 if k % 3 == 1 else 0.0)}

    _, o, grown = _run(SET, static, state, oracle, inputs, globals_fn, 8, {1, 2, 4, 8})
    assert grown > 0
