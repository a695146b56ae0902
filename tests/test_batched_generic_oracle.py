"""The batched oracle's user-UpdateConn path (the mean of the per-sample
writes, phases.py:484-533) and per-sample update_unit, pinned by the
reference's tests/test_batched.py assertions: for a linear rule the mean of
writes equals the exact batch-mean path (to rounding), and columns the rule
never writes, and dead slots, stay bit-identical across steps."""

from __future__ import annotations

import numpy as np

import batched_cases as bc
import nets
import plastax_amd as px
import update_conn_cases as uc
from oracle import batched as ob

AUX = px.FieldSpec.float32("test/aux", 0.1)


def _net(update, extra_conn=(), update_unit=None):
    attrs = dict(
        forward_pass=nets.SigmoidForward(), backward_pass=nets.SigmoidBackward(), loss=nets.MSELoss(),
        update_conn=update, extra_unit_fields=(nets.GRAD_PRE_ACT, nets.LOSS_GRAD),
        extra_conn_fields=tuple(extra_conn), batch_reduction=px.MeanFloatFirstRest())
    if update_unit is not None:
        attrs["update_unit"] = update_unit
    return type("BatchedGeneric", (px.Network,), attrs)


def _run(oracle, net, B, steps, seed=0, headroom=0.5):
    static, state = bc.build(net, [6, 5, 3], 0.9, seed=seed, device="cpu", headroom=headroom)
    o = nets.oracle_for(oracle, net, static, state)
    orc = ob.OracleBatch(o, B)
    xs, ys = bc.data(seed + 1, steps, B, 6, 3)
    for k in range(steps):
        orc.step(xs[k], ys[k])
    return o


def test_mean_of_writes_equals_the_exact_path_for_a_linear_rule(oracle) -> None:
    plain = _run(oracle, _net(uc.PlainSGD(0.2, nets.GRAD_PRE_ACT)), 4, 6)
    opt = px.optim.sgd(0.2, nets.GRAD_PRE_ACT)
    exact = _run(oracle, _net(opt.update_conn(), opt.state_fields), 4, 6)
    for a, b in zip(plain.conns, exact.conns):
        np.testing.assert_allclose(a["weight"], b["weight"], rtol=1e-5, atol=1e-6)


def test_mean_of_writes_leaves_unwritten_columns_and_dead_slots_bit_identical(oracle) -> None:
    net = _net(uc.PlainSGD(0.2, nets.GRAD_PRE_ACT), (AUX,))
    static, state = bc.build(net, [6, 5, 3], 0.9, seed=0, device="cpu", headroom=0.5)
    o = nets.oracle_for(oracle, net, static, state)
    before = [b[AUX.name].copy() for b in o.conns]
    dead_w = [b["weight"][b["dead"].astype(bool)].copy() for b in o.conns]
    assert any(w.size for w in dead_w)
    orc = ob.OracleBatch(o, 3)
    xs, ys = bc.data(1, 20, 3, 6, 3)
    for k in range(20):
        orc.step(xs[k], ys[k])
    for b, a0, w0 in zip(o.conns, before, dead_w):
        assert np.array_equal(b[AUX.name].view(np.uint32), a0.view(np.uint32))
        assert np.array_equal(b["weight"][b["dead"].astype(bool)].view(np.uint32), w0.view(np.uint32))
