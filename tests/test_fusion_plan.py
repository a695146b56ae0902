"""The prune-into-forward legality check (phases.py:1629-1848), on the host.

Mirrors the reference's cases (tests/test_prune_fusion.py): a predicate that
reads only edge columns and globals is fused; one that reads a field the
forward computes from its accumulator, or that a phase between the forward
and the prune writes (the loss seed, the update's WEIGHT), is not, and the
reason names the field; a field the forward writes from the globals and an
unwritten column is forwarded; prune_unit, a missing prune_conn and a field
forwarded from another forward-written field are refused.
"""

from __future__ import annotations

import numpy as np
import pytest

import nets
import plastax_amd as px
import plastax_amd.numpy as jnp
from plastax_amd.fusion import plan_prune_fusion

MARK = px.FieldSpec.float32("test/mark")
MASK = px.FieldSpec.float32("test/mask")


class HashPrune(px.PruneConn):
    """Reads only edge columns and the globals."""

    def predicate(self, u, c, cid, g):
        h = c[px.FROM_ID, cid] * jnp.int32(7) + c[px.TO_ID, cid] * jnp.int32(13) + g["step"]
        return (h % jnp.int32(11)) == jnp.int32(0)


class WeightPrune(px.PruneConn):
    def predicate(self, u, c, cid, g):
        return jnp.abs(c[px.WEIGHT, cid]) < g["tau"]


class ActivationPrune(px.PruneConn):
    def predicate(self, u, c, cid, g):
        return u[px.ACTIVATION, c[px.FROM_ID, cid]] < jnp.float32(-0.9)


class SeedPrune(px.PruneConn):
    def predicate(self, u, c, cid, g):
        return u[nets.LOSS_GRAD, c[px.TO_ID, cid]] > jnp.float32(10.0)


class MarkedPrune(px.PruneConn):
    def predicate(self, u, c, cid, g):
        return u[MARK, c[px.FROM_ID, cid]] > jnp.float32(0.5)


class MarkForward(px.ForwardPass):
    """Writes MARK from an unwritten column and the globals: forwarded."""

    combine = px.monoid.sum_

    def map(self, u, dst, src, c, cid, g):
        return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)), (MARK, u[MASK, i] * g["scale"]))


class SelfReadForward(MarkForward):
    """Writes MARK from ACTIVATION, itself written by the forward."""

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)), (MARK, u[px.ACTIVATION, i]))


class AccMarkForward(MarkForward):
    """Writes MARK from the accumulator."""

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)), (MARK, acc))


class KillUnit(px.PruneUnit):
    def predicate(self, u, i, g):
        return u[MASK, i] > jnp.float32(2.0)


G = {"step": np.int32(0), "tau": np.float32(0.01), "scale": np.float32(1.0)}


def _net(prune, *, forward=None, train=False, prune_unit=None):
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT)

    class Net(px.Network):
        forward_pass = forward or MarkForward()
        loss = nets.MSELoss() if train else None
        backward_pass = nets.TanhBackward() if train else None
        update_conn = opt.update_conn() if train else None
        prune_conn = prune
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD, MARK, MASK)
        extra_conn_fields = tuple(opt.state_fields) if train else ()
        unit_capacity = 40 if prune_unit is not None else None

    Net.prune_unit = prune_unit
    return Net


def _static(net):
    rng = np.random.default_rng(0)
    src = rng.integers(0, 8, 40).astype(np.int32)
    dst = rng.integers(8, 16, 40).astype(np.int32) + np.int32(8)
    static, _ = px.NetworkBuilder.from_edges(
        net, 32, src, dst, weights=rng.standard_normal(40).astype(np.float32), input_ids=np.arange(8),
        output_ids=np.arange(28, 32), globals_=G, capacity_headroom=0.5)
    return static


@pytest.mark.parametrize("train", [False, True])
def test_edge_column_predicate_is_fused(train: bool) -> None:
    net = _net(HashPrune(), train=train)
    plan = plan_prune_fusion(net, _static(net), G, engine="triton")
    assert plan.fused and plan.engine == "hip" and plan.forwarded == (), plan
    xla = plan_prune_fusion(net, _static(net), G, engine="xla")
    assert xla.fused and xla.engine == "xla", xla
    auto = plan_prune_fusion(net, _static(net), G)
    assert not auto.fused and "legal" in auto.reason, auto


def test_marked_predicate_forwards_the_field() -> None:
    net = _net(MarkedPrune(), train=True)
    plan = plan_prune_fusion(net, _static(net), G, engine="triton")
    assert plan.fused and plan.forwarded == (MARK.name,), plan


@pytest.mark.parametrize(
    ("prune", "forward", "train", "why"),
    [
        (ActivationPrune(), None, False, "accumulator"),
        (MarkedPrune(), AccMarkForward(), False, "accumulator"),
        (WeightPrune(), None, True, "weight"),
        (SeedPrune(), None, True, nets.LOSS_GRAD.name),
        (MarkedPrune(), SelfReadForward(), False, px.ACTIVATION.name),
    ],
)
def test_predicate_reading_a_written_field_is_not_fused(prune, forward, train, why) -> None:
    net = _net(prune, forward=forward, train=train)
    for engine in ("auto", "triton", "xla"):
        plan = plan_prune_fusion(net, _static(net), G, engine=engine)
        assert not plan.fused and why in plan.reason, plan


def test_weight_prune_without_update_conn_is_fused() -> None:
    net = _net(WeightPrune())
    assert plan_prune_fusion(net, _static(net), G, engine="triton").fused
    assert "legal" in plan_prune_fusion(net, _static(net), G).reason


def test_prune_unit_and_missing_prune_conn_are_not_fused() -> None:
    net = _net(HashPrune(), prune_unit=KillUnit())
    plan = plan_prune_fusion(net, _static(net), G)
    assert not plan.fused and "prune_unit" in plan.reason
    bare = _net(None)
    plan = plan_prune_fusion(bare, _static(bare), G)
    assert not plan.fused and plan.reason == "no prune_conn"


def test_unknown_engine_and_fuse_prune() -> None:
    net = _net(HashPrune())
    static = _static(net)
    with pytest.raises(ValueError, match="engine"):
        plan_prune_fusion(net, static, G, engine="sometimes")
    with pytest.raises(ValueError, match="fuse_prune"):
        px.make_step(net, static, fuse_prune="sometimes")
    step = px.make_step(net, static, fuse_prune="off")
    assert step.prune_fusion.requested == "off" and step.prune_fusion.plan is None
