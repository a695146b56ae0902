"""Losses outside MSE / softmax CE in the plan and the oracle (host only):
the TD error reading a fixed unit, checked against a float32 restatement in
the same operation order (bit for bit: a wrong unit or a dropped term fails
it); the weighted logistic loss against its float64 closed form; and the
tracer's refusals."""

from __future__ import annotations

import numpy as np
import pytest

import loss_cases as lc
import nets
import plastax_amd as px
from plastax_amd._expr import UnsupportedPolicyError
from plastax_amd._plan import compile_plan


def _setup(oracle, loss, seed=0):
    net = lc.make_net(loss)
    static, state = lc.build(net, seed=seed)
    o = nets.oracle_for(oracle, net, static, state)
    rng = np.random.default_rng(seed + 10)
    x = rng.standard_normal(len(static.input_ids)).astype(np.float32)
    o.units["activation"][np.asarray(static.input_ids)] = x
    o.units[lc.V_OLD.name][:] = rng.standard_normal(static.num_units).astype(np.float32)
    o.forward()
    return static, o, rng


def test_td_loss_reads_the_fixed_unit(oracle) -> None:
    gamma_unit = 3  # an input unit: its activation is the step's input
    static, o, rng = _setup(oracle, lc.TdLoss(gamma_unit))
    plan = compile_plan(lc.make_net(lc.TdLoss(gamma_unit)), static)
    assert list(plan.loss.program.fixed_at.values()) == [gamma_unit]
    out = np.asarray(static.output_ids)
    t = lc.targets_for(o.plan.net.loss, rng, out.size)
    val = o.loss(t)
    act, vo = o.units["activation"], o.units[lc.V_OLD.name]
    gamma = act[gamma_unit]
    delta = (t + gamma * act[out]) - vo[out]  # float32, the traced order
    want = np.float32(0.0)
    for d in delta:  # one piece of <= 256 terms: a left fold from +0.0
        want = np.float32(want + np.float32(np.float32(0.5) * d) * d)
    want = np.float32(np.float32(0.0) + want)
    assert np.float32(val).view(np.uint32) == want.view(np.uint32)
    assert np.array_equal(o.units[nets.LOSS_GRAD.name][out].view(np.uint32), delta.view(np.uint32))


def test_weighted_logistic_loss_matches_its_closed_form(oracle) -> None:
    loss = lc.WeightedLogisticLoss(2.5)
    static, o, rng = _setup(oracle, loss, seed=1)
    out = np.asarray(static.output_ids)
    t = lc.targets_for(loss, rng, out.size)
    val = o.loss(t)
    z = o.units["activation"][out].astype(np.float64)
    w, t64 = 2.5, t.astype(np.float64)
    scale = 1 + t64 * (w - 1)
    exact = np.sum(scale * (np.maximum(z, 0) + np.log1p(np.exp(-np.abs(z)))) - w * t64 * z)
    assert abs(float(val) - exact) <= 1e-5 * max(1.0, abs(exact))
    seed = scale / (1 + np.exp(-z)) - w * t64
    assert np.max(np.abs(o.units[nets.LOSS_GRAD.name][out] - seed)) <= 1e-6


def test_fixed_unit_reads_are_for_the_loss_only() -> None:
    class Peek(nets.TanhForward):
        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((px.ACTIVATION, acc + u[px.ACTIVATION, px.UnitIdx(np.int32(0))]))

    net = lc.make_net(lc.TdLoss(0))
    net.forward_pass = Peek()
    static, _ = lc.build(net, seed=2)
    with pytest.raises(UnsupportedPolicyError, match="fixed unit"):
        compile_plan(net, static)
    far = lc.make_net(lc.TdLoss(10**6))
    static2, _ = lc.build(far, seed=2)
    with pytest.raises(UnsupportedPolicyError, match="reads unit"):
        compile_plan(far, static2)
