"""Product maps on the device (map_term in the kernels): constant and lone
factors in the forward, the tiled backward fused with the update, the churn
layout's backward lists and the batched kernels, against the oracle bit for
bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import batched_cases as bc
import nets
import plastax_amd as px
import plastax_amd.numpy as jnp
from plastax_amd import synth
from test_gpu_parity import _equal, assert_same_state
from test_maps import INDEG, OUTDEG, WSUM, CountIn, CountOut, WeightSum, degree_net

pytestmark = pytest.mark.gpu


class HalfInputForward(px.ForwardPass):
    """tanh of half the unweighted sum of the inputs (w factor constant)."""

    combine = px.monoid.sum_

    def map(self, u, dst, src, c, cid, g):
        return jnp.float32(0.5) * u[px.ACTIVATION, src]

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)))


class DoubledWeightBackward(px.BackwardPass):
    """A backward whose map drops the grad (unit factor constant)."""

    combine = px.monoid.sum_

    def map(self, u, src, dst, c, cid, g):
        return c[px.WEIGHT, cid] * 2.0

    def apply(self, u, i, g, acc):
        a = u[px.ACTIVATION, i]
        return px.UnitWrite.of((nets.GRAD_PRE_ACT, (acc * jnp.float32(0.01) + u[nets.LOSS_GRAD, i])
                                * (jnp.float32(1.0) - a * a)))


def _compare(oracle, net, static, state, steps, inputs, tile=None, mode=None):
    o = nets.oracle_for(oracle, net, static, state)
    o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
    step = px.make_step(net, static)
    if mode is not None:
        step.arena_mode = mode
    if tile is not None:
        step.tile = tile
        o.tile = tile
    if step.backward_order == "slot":
        o.tile = None
    for k in range(1, steps + 1):
        x, t = inputs(k)
        print(f"map step {k} net={net.__name__}", flush=True)
        res = step(state, px.StepInputs(x, t))
        state = res.state
        lo = o.step(x, t)
        torch.cuda.synchronize()
        assert_same_state(static, state, o, f"step {k}")
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at {k}"
    return state, o


@pytest.mark.parametrize("forward", [CountIn(), WeightSum()])
def test_degree_counts_on_the_tiled_layout(oracle, forward) -> None:
    """In-degree / in-weight forward and out-degree backward over a Zipf net
    (hot and cold sources, small tiles): every column, and the counts equal
    the live edge counts."""
    e = synth.c2_topological(seed=9, scale=256, layers=5)
    net = degree_net(forward, px.Propagation.TOPOLOGICAL)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cuda")
    x = np.zeros(e.input_ids.size, np.float32)
    state, o = _compare(oracle, net, static, state, 2, lambda k: (x, None), tile=256)
    out = state.units[OUTDEG.name].cpu().numpy()
    level = state.units["level"].cpu().numpy()
    want = np.bincount(e.src, minlength=e.num_units).astype(np.float32)
    sel = level > 0
    assert np.array_equal(out[sel], want[sel])


def test_constant_factors_with_training(oracle) -> None:
    """A trained net whose forward map has a constant connection factor and
    whose backward map has a constant unit factor (the fused backward +
    update keeps updating WEIGHT)."""
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT)
    net = nets.make_trained_net("ConstFactors", HalfInputForward(), DoubledWeightBackward(), opt,
                                px.Propagation.TOPOLOGICAL)
    e = synth.c2_topological(seed=2, scale=512, layers=4)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cuda")
    rng = np.random.default_rng(3)
    xs = rng.standard_normal((4, e.input_ids.size)).astype(np.float32)
    _compare(oracle, net, static, state, 4, lambda k: (xs[k - 1], np.tanh(xs[k - 1][::-1]).astype(np.float32)))


class Propose(px.ProposeAddConn):
    proposer = "per_unit"
    proposals_per_proposer = 2
    max_new_per_level = 10
    max_level_gap = 1 << 20

    def propose(self, u, i, j, g, rng):
        return jnp.asarray(i, jnp.int32), rng.uniform_int(600).astype(jnp.int32), rng.uniform()

    def init(self, u, src, dst, g):
        return px.ConnWrite.of((px.WEIGHT, jnp.float32(0.05)))


def test_out_degree_on_the_churn_layout(oracle) -> None:
    """A growing PIPELINE reservoir (growth every step: the churn layout,
    backward lists) counting its units' out-degree each step."""

    class Reservoir(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = CountOut()
        add_conn = Propose()
        extra_unit_fields = (OUTDEG,)
        propagation = px.Propagation.PIPELINE

    rng = np.random.default_rng(21)
    n = 600
    src = rng.integers(0, n, 3000).astype(np.int32)
    dst = rng.integers(0, n, 3000).astype(np.int32)
    keep = src != dst
    src, dst = src[keep], dst[keep]
    w = (rng.standard_normal(src.size) * 0.2).astype(np.float32)
    static, state = px.NetworkBuilder.from_edges(
        Reservoir, n, src, dst, weights=w, input_ids=np.arange(16), output_ids=np.arange(n - 4, n),
        globals_=None, capacity_headroom=1.0, device="cuda")
    assert px.make_step(Reservoir, static).backward_order == "slot"
    xs = rng.standard_normal((5, 16)).astype(np.float32)
    _compare(oracle, Reservoir, static, state, 5, lambda k: (xs[k - 1], None))


@pytest.mark.parametrize("B", [4, 256])
def test_batched_lone_and_constant_maps(oracle, B: int) -> None:
    """make_step(batch_size=B) with a lone-field forward map and a constant
    backward map, levels wide enough (512 rows) for the one-wave row kernels
    at B = 256."""
    from oracle import batched as ob

    class Lone(px.ForwardPass):
        combine = px.monoid.sum_

        def map(self, u, dst, src, c, cid, g):
            return u[px.ACTIVATION, src]

        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc * jnp.float32(0.05))))

    class Const(px.BackwardPass):
        combine = px.monoid.sum_

        def map(self, u, src, dst, c, cid, g):
            return jnp.float32(0.25)

        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((nets.GRAD_PRE_ACT, acc + u[nets.LOSS_GRAD, i]))

    opt = px.optim.sgd(1e-2, nets.GRAD_PRE_ACT)

    class Net(px.Network):
        forward_pass = Lone()
        backward_pass = Const()
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        batch_reduction = px.MeanFloatFirstRest()

    layers = [40, 512, 512, 8]
    static, state = bc.build(Net, layers, 0.05, seed=5, device="cuda")
    o = nets.oracle_for(oracle, Net, static, state)
    orc = ob.OracleBatch(o, B)
    step = px.make_step(Net, static, batch_size=B)
    xs, ys = bc.data(6, 2, B, layers[0], layers[-1])
    for k in range(2):
        print(f"batched map step {k} B={B}", flush=True)
        res = step(state, px.StepInputs(xs[k], ys[k]))
        state = res.state
        lo = orc.step(xs[k], ys[k])
        torch.cuda.synchronize()
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at step {k}"
        assert_same_state(static, state, o, f"step {k}")
