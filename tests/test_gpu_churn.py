"""The churn layout (plastax_amd/_churn.py): an arena rebuilt on the device
after every structural change, whose backward folds each source's live
out-edges in logical slot order -- the reference's own scatter order, the
oracle's `tile=None` fold. Device vs oracle, bit for bit: every unit and
connection column, the loss and the structural flags, step after step."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import batched_cases as bc
import nets
import plastax_amd as px
import plastax_amd.numpy as jnp
from test_gpu_parity import _equal, assert_same_state

pytestmark = pytest.mark.gpu


class TauPrune(px.PruneConn):
    def predicate(self, u, c, cid, g):
        return jnp.abs(c[px.WEIGHT, cid]) < g["tau"]


class Propose(px.ProposeAddConn):
    proposer = "per_unit"
    proposals_per_proposer = 3
    max_new_per_level = 8
    max_level_gap = 1 << 20

    def __init__(self, n: int) -> None:
        self.n = n

    def propose(self, u, i, j, g, rng):
        dst = rng.uniform_int(self.n).astype(jnp.int32)
        return jnp.asarray(i, jnp.int32), dst, rng.uniform() + jnp.abs(u[px.ACTIVATION, i])

    def init(self, u, src, dst, g):
        return px.ConnWrite.of((px.WEIGHT, jnp.float32(0.03)))


class Deeper(px.ScoreAddConn):
    candidates = "shortlist_per_level"
    shortlist_size = 12
    direction = "deeper"
    dedupe_live = True
    max_new_per_level = 12

    def score(self, u, src, dst, g):
        return jnp.abs(u[px.ACTIVATION, src] * u[nets.GRAD_PRE_ACT, dst])

    def importance(self, u, i, g):
        return jnp.abs(u[nets.GRAD_PRE_ACT, i]) + jnp.abs(u[px.ACTIVATION, i])

    def init(self, u, src, dst, g):
        return px.ConnWrite.of((px.WEIGHT, jnp.float32(0.0)))


def _net(pipeline: bool, grow, opt):
    class Net(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        prune_conn = TauPrune()
        add_conn = grow
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        extra_conn_fields = tuple(opt.state_fields)
        propagation = px.Propagation.PIPELINE if pipeline else px.Propagation.TOPOLOGICAL

    return Net


def _steps(oracle, net, static, state, mode: str, steps: int, seed: int):
    o = nets.oracle_for(oracle, net, static, state)
    o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
    step = px.make_step(net, static)
    step.arena_mode = mode
    if step.backward_order == "slot":
        o.tile = None
    rng = np.random.default_rng(seed)
    n_in, n_out = len(static.input_ids), len(static.output_ids)
    teacher = (rng.standard_normal((n_out, n_in)) * 0.3).astype(np.float32)
    grown = 0
    for k in range(1, steps + 1):
        g = {"tau": np.float32(0.004 * (k % 3))}
        state.globals_, o.globals_ = g, g
        x = rng.standard_normal(n_in).astype(np.float32)
        t = np.tanh(teacher @ x).astype(np.float32)
        print(f"churn-layout step {k} mode={mode}", flush=True)
        res = step(state, px.StepInputs(x, t))
        state = res.state
        lo = o.step(x, t)
        assert (state.grown, state.overflow, state.needs_resort, state.tail_start) == (
            o.grown, o.overflow, o.needs_resort, o.tail_start), f"flags at step {k}"
        grown += state.grown
        torch.cuda.synchronize()
        assert_same_state(static, state, o, f"step {k}")
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at step {k}"
    return grown


def test_reservoir_growth_every_step(oracle) -> None:
    rng = np.random.default_rng(11)
    n = 1500
    src = rng.integers(0, n, 12000).astype(np.int32)
    dst = rng.integers(0, n, 12000).astype(np.int32)
    keep = src != dst
    src, dst = src[keep], dst[keep]
    w = (rng.standard_normal(src.size) * 0.3).astype(np.float32)
    net = _net(True, Propose(n), px.optim.adam(1e-2, nets.GRAD_PRE_ACT))
    static, state = px.NetworkBuilder.from_edges(
        net, n, src, dst, weights=w, input_ids=np.arange(32), output_ids=np.arange(n - 8, n),
        globals_={"tau": np.float32(0.0)}, capacity_headroom=1.0, device="cuda")
    assert px.make_step(net, static).backward_order == "slot"
    assert _steps(oracle, net, static, state, "auto", 8, 1) > 0


@pytest.mark.parametrize("mode", ["churn", "tiled"])
def test_layered_growth_every_step_both_layouts(oracle, mode: str) -> None:
    net = _net(False, Deeper(), px.optim.sgd(0.05, nets.GRAD_PRE_ACT))
    static, state = bc.build(net, [24, 60, 50, 8], 0.25, skip=0.05, seed=12, device="cuda", headroom=0.5)
    state.globals_ = {"tau": np.float32(0.0)}
    assert _steps(oracle, net, static, state, mode, 6, 2) > 0


def test_forced_churn_layout_without_structure(oracle) -> None:
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT)
    net = bc.tanh_mse_net(opt)
    static, state = bc.build(net, [30, 64, 48, 10], 0.3, skip=0.1, seed=13, device="cuda")
    o = nets.oracle_for(oracle, net, static, state)
    o.tile = None
    step = px.make_step(net, static)
    step.arena_mode = "churn"
    xs, ys = bc.data(3, 5, 1, 30, 10)
    for k in range(5):
        res = step(state, px.StepInputs(xs[k, 0], ys[k, 0]))
        state = res.state
        lo = o.step(xs[k, 0], ys[k, 0])
        torch.cuda.synchronize()
        assert_same_state(static, state, o, f"step {k}")
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at step {k}"
