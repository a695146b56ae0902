"""Network classes and helpers shared by the tests.

The policies mirror the reference's own test policies
(tests/test_parity_goldens.py:131-228, examples/mlp_xor.py:46-124) written
against plastax_amd's jnp-style API.
"""

from __future__ import annotations

import json
import pathlib
from typing import Any

import numpy as np

import plastax_amd as px
import plastax_amd.numpy as jnp
from plastax_amd import synth
from plastax_amd.state import column_to_numpy

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"

GRAD_PRE_ACT = px.FieldSpec.float32("grad_pre_act")
LOSS_GRAD = px.FieldSpec.float32("loss_grad")


def load_golden(name: str) -> dict[str, Any]:
    return json.loads((GOLDEN / name).read_text())


class _WeightedSumMap:
    combine = px.monoid.sum_

    def map(self, u, dst, src, c, cid, g):
        return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]


class ReluForward(_WeightedSumMap, px.ForwardPass):
    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, jnp.maximum(acc, jnp.float32(0.0))))


class LinearForward(_WeightedSumMap, px.ForwardPass):
    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, acc))


class TanhForward(_WeightedSumMap, px.ForwardPass):
    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)))


class SigmoidForward(_WeightedSumMap, px.ForwardPass):
    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, px.nn.sigmoid(acc)))


class MaxForward(px.ForwardPass):
    combine = px.monoid.max_

    def map(self, u, dst, src, c, cid, g):
        return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)))


class _GradMap:
    combine = px.monoid.sum_

    def map(self, u, src, dst, c, cid, g):
        return c[px.WEIGHT, cid] * u[GRAD_PRE_ACT, dst]


class ReluBackward(_GradMap, px.BackwardPass):
    def apply(self, u, i, g, acc):
        gate = jnp.where(u[px.ACTIVATION, i] > 0, jnp.float32(1.0), jnp.float32(0.0))
        return px.UnitWrite.of((GRAD_PRE_ACT, (acc + u[LOSS_GRAD, i]) * gate))


class TanhBackward(_GradMap, px.BackwardPass):
    def apply(self, u, i, g, acc):
        a = u[px.ACTIVATION, i]
        return px.UnitWrite.of((GRAD_PRE_ACT, (acc + u[LOSS_GRAD, i]) * (jnp.float32(1.0) - a * a)))


class SigmoidBackward(_GradMap, px.BackwardPass):
    def apply(self, u, i, g, acc):
        a = u[px.ACTIVATION, i]
        return px.UnitWrite.of(
            (GRAD_PRE_ACT, (acc + u[LOSS_GRAD, i]) * a * (jnp.float32(1.0) - a))
        )


class MSELoss(px.Loss):
    seed_field = LOSS_GRAD

    def calculate_loss(self, u, outputs, targets, g):
        diff = u.gather(px.ACTIVATION, outputs) - targets
        return jnp.sum(jnp.float32(0.5) * diff * diff), diff


class ReluMlpNet(px.Network[None]):
    forward_pass = ReluForward()
    backward_pass = ReluBackward()
    loss = MSELoss()
    extra_unit_fields = (GRAD_PRE_ACT, LOSS_GRAD)
    propagation = px.Propagation.TOPOLOGICAL


class ReluPipelineNet(px.Network[None]):
    forward_pass = ReluForward()
    propagation = px.Propagation.PIPELINE


class SoftmaxNet(px.Network[None]):
    forward_pass = LinearForward()
    loss = px.SoftmaxCrossEntropyLoss(LOSS_GRAD)
    extra_unit_fields = (LOSS_GRAD,)
    propagation = px.Propagation.TOPOLOGICAL


def make_trained_net(name: str, forward, backward, optimizer, propagation, loss=None):
    """A Network class with the given policies and optimizer bundle."""
    attrs = dict(
        forward_pass=forward,
        backward_pass=backward,
        loss=loss if loss is not None else MSELoss(),
        update_conn=optimizer.update_conn(),
        extra_unit_fields=(GRAD_PRE_ACT, LOSS_GRAD),
        extra_conn_fields=tuple(optimizer.state_fields),
        propagation=propagation,
    )
    return type(name, (px.Network,), attrs)


def golden_edges(doc: dict[str, Any]) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    e = doc["initial_edges"]
    return (
        np.asarray([x["src"] for x in e], np.int32),
        np.asarray([x["dst"] for x in e], np.int32),
        np.asarray([x["fields"]["weight"] for x in e], np.float32),
    )


def build_golden(net, doc: dict[str, Any], device: str = "cpu"):
    """The golden's network through from_edges (every golden lists its edges)."""
    src, dst, w = golden_edges(doc)
    n_in = doc["network"]["input_dim"]
    n = n_in + sum(doc["network"]["layers"])
    last = doc["network"]["layers"][-1]
    return px.NetworkBuilder.from_edges(
        net, n, src, dst, weights=w,
        input_ids=list(range(n_in)), output_ids=list(range(n - last, n)),
        globals_=None, device=device,
    )


def host_units(static, state) -> dict[str, np.ndarray]:
    return {
        s.name: np.array(column_to_numpy(state.units[s.name], s), copy=True, order="C")
        for s in static.unit_fields
    }


def host_conns(static, state) -> list[dict[str, np.ndarray]]:
    specs = {s.name: s for s in static.conn_fields}
    return [
        {n: np.array(column_to_numpy(b[n], specs[n]), copy=True, order="C") for n in specs}
        for b in state.conns
    ]


def oracle_for(ox, net, static, state, **kw):
    from plastax_amd._plan import compile_plan

    plan = compile_plan(net, static)
    return ox.OracleNet(static, host_units(static, state), host_conns(static, state), plan,
                        state.globals_, **kw)


def hub_edges(seed: int, widths: tuple[int, ...] = (64, 256, 512, 16), fan: tuple[int, ...] = (4, 6, 12),
              hubs: int = 2) -> synth.EdgeList:
    """A layered net whose first `hubs` units of every layer feed every unit
    of the next: with short rows a backward tile holds many destinations,
    so a hub's (tile, source) group runs over many ranks."""
    rng = np.random.default_rng(seed)
    base = np.concatenate([[0], np.cumsum(widths)])
    src, dst = [], []
    for l in range(len(widths) - 1):
        for j in range(widths[l + 1]):
            others = rng.choice(np.arange(hubs, widths[l]), size=fan[l] - hubs, replace=False)
            for i in np.concatenate([np.arange(hubs), others]):
                src.append(base[l] + i)
                dst.append(base[l + 1] + j)
    src = np.asarray(src, dtype=np.int32)
    dst = np.asarray(dst, dtype=np.int32)
    w = (rng.standard_normal(src.size) * 0.3).astype(np.float32)
    return synth.EdgeList(int(base[-1]), src, dst, w, np.arange(widths[0], dtype=np.int32),
                          np.arange(base[-2], base[-1], dtype=np.int32))
