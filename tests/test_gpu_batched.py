"""Batched steps on the device (make_step(batch_size=B), step.py:359-468):
the forward / backward per sample, the exact batch-mean update, the batch
reductions and the batch-mean loss must equal the batched oracle
(oracle/batched.py) bit for bit -- every unit column, every connection
column and the loss, at every step."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import batched_cases as bc
import nets
import plastax_amd as px
from test_gpu_parity import _equal, assert_same_state

pytestmark = pytest.mark.gpu


def _run(oracle, net, layers, keep, skip, B, steps, seed=0, onehot=False, headroom=0.0, check=None):
    from oracle import batched as ob

    static, state = bc.build(net, layers, keep, skip=skip, seed=seed, device="cuda", headroom=headroom)
    o = nets.oracle_for(oracle, net, static, state)
    o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
    orc = ob.OracleBatch(o, B)
    step = px.make_step(net, static, batch_size=B)
    xs, ys = bc.data(seed + 1, steps, B, layers[0], layers[-1], onehot=onehot)
    for k in range(steps):
        print(f"batched step {k} B={B} layers={layers}", flush=True)
        res = step(state, px.StepInputs(xs[k], ys[k]))
        state = res.state
        lo = orc.step(xs[k], ys[k])
        if check is not None:
            check(k, state, o)
        torch.cuda.synchronize()
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at step {k}: {float(res.loss)} vs {lo}"
        assert_same_state(static, state, o, f"step {k}")
    return state, o


@pytest.mark.parametrize("B", [1, 3, 16, 70])
def test_tanh_mse_adam_with_skip_edges(oracle, B: int) -> None:
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT)
    _run(oracle, bc.tanh_mse_net(opt), [20, 48, 40, 8], 0.3, 0.05, B, 4)


@pytest.mark.parametrize("rule", ["sgd", "momentum", "rmsprop", "adamw"])
def test_every_rule_on_the_batch_mean(oracle, rule: str) -> None:
    make = {
        "sgd": lambda: px.optim.sgd(0.05, nets.GRAD_PRE_ACT),
        "momentum": lambda: px.optim.momentum(0.05, 0.9, nets.GRAD_PRE_ACT),
        "rmsprop": lambda: px.optim.rmsprop(1e-3, nets.GRAD_PRE_ACT),
        "adamw": lambda: px.optim.adamw(1e-3, nets.GRAD_PRE_ACT, weight_decay=1e-2),
    }[rule]
    _run(oracle, bc.tanh_mse_net(make()), [16, 32, 8], 0.4, 0.0, 8, 3, seed=2)


def test_dense_tiles_are_split(oracle) -> None:
    """90 % keep: a 64 x 64-unit tile of the batched update holds ~3,700
    edges, so it is cut into several tiles of at most 1,024 edges (samples
    in two chunks of 64, the last one short)."""
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT)
    _run(oracle, bc.tanh_mse_net(opt), [64, 128, 64, 8], 0.9, 0.0, 100, 2, seed=6)


def test_c3_shaped_softmax_batch(oracle) -> None:
    """C3's shape scaled down: 784-128-128-10 at 10 % keep, B = 256,
    softmax cross-entropy, Adam."""
    opt = px.optim.adam(1e-3, nets.GRAD_PRE_ACT)
    _run(oracle, bc.softmax_net(opt), [784, 128, 128, 10], 0.1, 0.0, 256, 2, seed=4, onehot=True)


@pytest.mark.parametrize("B", [64, 256])
def test_long_rows_cross_the_staged_chunks(oracle, B: int) -> None:
    """Few rows with thousands of in- and out-edges (3,000 -> 6 -> 4 at 60 %
    keep: ~1,800 in-edges per hidden row, ~3,600 edges per output's backward
    row set): the workgroup-per-row kernels stage a row's positions in LDS
    1,024 at a time, so each row's fold crosses chunk boundaries; with
    skip edges and dead slots from the builder's headroom."""
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT)
    _run(oracle, bc.tanh_mse_net(opt), [3000, 6, 4], 0.6, 0.05, B, 2, seed=9, headroom=0.25)


@pytest.mark.parametrize("B", [256, 132])
def test_wide_levels_run_the_one_wave_row_kernels(oracle, B: int) -> None:
    """Levels of 512 rows at a batch that is a multiple of 4 and >= 128: the
    forward of both hidden levels and the backward of both reduced buckets
    take the one-wave-per-row kernels (k_forward_batch4, k_backward_batch4;
    plx_forward_batch / plx_backward_batch dispatch them for B % 4 == 0,
    B >= 128 and >= 256 rows). B = 132 leaves 31 lanes of each wave without
    samples. Softmax cross-entropy and Adam, as at C3."""
    opt = px.optim.adam(1e-3, nets.GRAD_PRE_ACT)
    _run(oracle, bc.softmax_net(opt), [784, 512, 512, 10], 0.1, 0.0, B, 2, seed=7, onehot=True)


def test_wide_levels_with_the_max_monoid(oracle) -> None:
    """The same one-wave-per-row kernels folding with the max monoid in the
    forward (skip edges carry accumulators across levels)."""
    opt = px.optim.adam(1e-3, nets.GRAD_PRE_ACT)

    class Net(px.Network):
        forward_pass = nets.MaxForward()
        backward_pass = nets.TanhBackward()
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        extra_conn_fields = tuple(opt.state_fields)
        batch_reduction = px.MeanFloatFirstRest()

    _run(oracle, Net, [64, 384, 320, 8], 0.2, 0.02, 256, 2, seed=8)


def test_structural_phases_run_once_per_batch(oracle) -> None:
    """tests/test_batched.py:189-229: prune and growth see the reduced state,
    once per batched step."""

    class TauPrune(px.PruneConn):
        def predicate(self, u, c, cid, g):
            return px.numpy.abs(c[px.WEIGHT, cid]) < np.float32(0.02)

    class Grow(px.ScoreAddConn):
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

    opt = px.optim.sgd(0.05, nets.GRAD_PRE_ACT)

    class Net(bc.tanh_mse_net(opt)):
        prune_conn = TauPrune()
        add_conn = Grow()

    grown = []

    def check(k, state, o):
        assert (state.grown, state.overflow) == (o.grown, o.overflow), f"flags at step {k}"
        grown.append(state.grown)

    _run(oracle, Net, [16, 40, 30, 6], 0.3, 0.0, 5, 4, seed=5, headroom=0.5, check=check)
    assert sum(grown) > 0


def test_policy_and_shape_errors() -> None:
    opt = px.optim.sgd(0.05, nets.GRAD_PRE_ACT)

    class Partial(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        batch_reduction = px.FieldReductions({px.ACTIVATION: px.Reduction.MEAN,
                                              nets.LOSS_GRAD: px.Reduction.MEAN})

    static, state = bc.build(Partial, [6, 5, 3], 1.0, device="cuda")
    step = px.make_step(Partial, static, batch_size=2)
    xs, ys = bc.data(0, 1, 2, 6, 3)
    with pytest.raises(ValueError, match=r"'grad_pre_act'.*backward_pass.*not declare"):
        step(state, px.StepInputs(xs[0], ys[0]))
    net = bc.tanh_mse_net(opt)
    static, state = bc.build(net, [6, 5, 3], 1.0, device="cuda")
    step = px.make_step(net, static, batch_size=4)
    with pytest.raises(ValueError, match="inputs must be"):
        step(state, px.StepInputs(xs[0], ys[0]))


def test_sum_first_and_mean_reductions(oracle) -> None:
    """reduce_batch_units (phases.py:298-332) in all three modes: the input
    scatter's and forward's ACTIVATION summed, the loss seed from sample 0,
    the backward's grads averaged."""
    opt = px.optim.sgd(0.05, nets.GRAD_PRE_ACT)

    class Net(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        batch_reduction = px.FieldReductions({px.ACTIVATION: px.Reduction.SUM,
                                              nets.LOSS_GRAD: px.Reduction.FIRST,
                                              nets.GRAD_PRE_ACT: px.Reduction.MEAN})

    _run(oracle, Net, [10, 24, 6], 0.5, 0.0, 5, 3, seed=6)
