"""Batched steps with a user UpdateConn (the mean of the per-sample writes)
and with update_unit (per sample, reduced by batch_reduction), against the
batched oracle bit for bit, at batch sizes that leave lanes idle and at the
one-wave row kernels' B = 256."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import batched_cases as bc
import nets
import plastax_amd as px
import plastax_amd.numpy as jnp
import update_conn_cases as uc
from test_gpu_parity import _equal, assert_same_state

pytestmark = pytest.mark.gpu

AUX = px.FieldSpec.float32("test/aux", 0.1)
NUDGE = px.FieldSpec.float32("nudge", 0.0)
COUNT = px.FieldSpec.int32("count", 0)


class Nudge(px.UpdateUnit):
    """A per-sample unit rule: a decaying trace of the activation and an
    integer counter bumped where the unit fired."""

    def update(self, u, i, g):
        fired = (u[px.ACTIVATION, i] > jnp.float32(0.5)).astype(jnp.int32)
        return px.UnitWrite.of((NUDGE, u[NUDGE, i] * jnp.float32(0.5) + u[px.ACTIVATION, i]),
                               (COUNT, u[COUNT, i] + fired))


class HebbNoisy(px.UpdateConn):
    """A nonlinear rule writing two float columns from both passes."""

    def incoming(self, u, dst, src, c, cid, g):
        h = jnp.tanh(u[px.ACTIVATION, dst] * u[px.ACTIVATION, src] * jnp.float32(3.0))
        return px.ConnWrite.of((px.WEIGHT, c[px.WEIGHT, cid] + jnp.float32(0.01) * h))

    def outgoing(self, u, src, dst, c, cid, g):
        return px.ConnWrite.of((AUX, c[AUX, cid] * jnp.float32(0.9) + jnp.abs(c[px.WEIGHT, cid])))


def _net(update, extra_conn=(), update_unit=None, extra_unit=()):
    attrs = dict(
        forward_pass=nets.TanhForward(), backward_pass=nets.TanhBackward(), loss=nets.MSELoss(),
        update_conn=update, extra_unit_fields=(nets.GRAD_PRE_ACT, nets.LOSS_GRAD, *extra_unit),
        extra_conn_fields=tuple(extra_conn), batch_reduction=px.MeanFloatFirstRest())
    if update_unit is not None:
        attrs["update_unit"] = update_unit
    return type("BatchedGeneric", (px.Network,), attrs)


def _run(oracle, net, layers, keep, B, steps, seed=0):
    from oracle import batched as ob

    static, state = bc.build(net, layers, keep, skip=0.05, seed=seed, device="cuda", headroom=0.3)
    o = nets.oracle_for(oracle, net, static, state)
    orc = ob.OracleBatch(o, B)
    step = px.make_step(net, static, batch_size=B)
    xs, ys = bc.data(seed + 1, steps, B, layers[0], layers[-1])
    for k in range(steps):
        print(f"batched generic step {k} B={B} net={net.__name__}", flush=True)
        res = step(state, px.StepInputs(xs[k], ys[k]))
        state = res.state
        lo = orc.step(xs[k], ys[k])
        torch.cuda.synchronize()
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at step {k}"
        assert_same_state(static, state, o, f"step {k}")


@pytest.mark.parametrize("B", [1, 3, 16])
def test_mean_of_writes_plain_sgd(oracle, B: int) -> None:
    _run(oracle, _net(uc.PlainSGD(0.1, nets.GRAD_PRE_ACT), (AUX,)), [12, 40, 30, 6], 0.3, B, 3)


def test_mean_of_writes_nonlinear_two_pass_rule(oracle) -> None:
    _run(oracle, _net(HebbNoisy(), (AUX,)), [12, 40, 30, 6], 0.3, 5, 3, seed=4)


@pytest.mark.parametrize("B", [3, 256])
def test_update_unit_per_sample(oracle, B: int) -> None:
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT)
    net = _net(opt.update_conn(), opt.state_fields, Nudge(), (NUDGE, COUNT))
    layers = [16, 256, 256, 6] if B == 256 else [12, 40, 30, 6]
    _run(oracle, net, layers, 0.1 if B == 256 else 0.3, B, 2, seed=2)
