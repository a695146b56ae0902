"""Losses after the reference's examples, beyond MSE and softmax CE: the
extreme-classification loss of examples/xmc.py:150-178 (log1p, exp, abs,
sigmoid, a positive-class weight) and the TD error of
examples/swifttd.py:365-392, which reads one unit fixed at construction
(``u[ACTIVATION, UnitIdx(gamma_unit)]``) besides the outputs' own fields.
Shared by the oracle tests and the device tests."""

from __future__ import annotations

import numpy as np

import batched_cases as bc
import nets
import plastax_amd as px
import plastax_amd.nn as pnn
import plastax_amd.numpy as jnp

V_OLD = px.FieldSpec.float32("test/v_old", 0.25)


class WeightedLogisticLoss(px.Loss):
    """sum(scale * (max(z, 0) + log1p(exp(-|z|))) - w * t * z), seed
    scale * sigmoid(z) - w * t with scale = 1 + t * (w - 1)."""

    seed_field = nets.LOSS_GRAD

    def __init__(self, pos_weight: float = 2.0) -> None:
        self.pos_weight = pos_weight

    def calculate_loss(self, u, outputs, targets, g):
        z = u.gather(px.ACTIVATION, outputs)
        w = jnp.float32(self.pos_weight)
        scale = jnp.float32(1.0) + targets * (w - jnp.float32(1.0))
        loss = scale * (jnp.maximum(z, jnp.float32(0.0)) + jnp.log1p(jnp.exp(-jnp.abs(z)))) - w * targets * z
        return jnp.sum(loss), scale * pnn.sigmoid(z) - w * targets


class TdLoss(px.Loss):
    """delta = t + gamma * v - v_old, gamma the activation of one fixed unit."""

    seed_field = nets.LOSS_GRAD

    def __init__(self, gamma_unit: int) -> None:
        self.gamma_unit = gamma_unit

    def calculate_loss(self, u, outputs, targets, g):
        v = u.gather(px.ACTIVATION, outputs)
        v_old = u.gather(V_OLD, outputs)
        gamma = u[px.ACTIVATION, px.UnitIdx(jnp.int32(self.gamma_unit))]
        delta = targets + gamma * v - v_old
        return jnp.sum(jnp.float32(0.5) * delta * delta), delta


def make_net(loss, *, batched: bool = False, opt=None):
    opt = opt or px.optim.adam(1e-2, nets.GRAD_PRE_ACT)

    class Net(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        update_conn = opt.update_conn()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD, V_OLD)
        extra_conn_fields = tuple(opt.state_fields)

    Net.loss = loss
    if batched:
        Net.batch_reduction = px.MeanFloatFirstRest()
    return Net


LAYERS = [20, 48, 40, 12]


def build(net, *, seed: int, device: str = "cpu"):
    return bc.build(net, LAYERS, 0.3, skip=0.05, seed=seed, device=device)


def targets_for(loss, rng, shape):
    if isinstance(loss, WeightedLogisticLoss):
        return (rng.random(shape) < 0.3).astype(np.float32)  # labels in {0, 1}
    return (rng.standard_normal(shape) * 0.5).astype(np.float32)
