"""User UpdateConn policies (not optim bundles) and the known answers of the
reference's tests/test_update_conn.py: an order probe (incoming writes a
marker, outgoing adds 1000 to the current weight: every live edge ends at
-123.5 + 1000), endpoint probes (weight <- activation[dst] - activation[src]
from either pass), dead slots untouched, every TOPOLOGICAL bucket swept."""

from __future__ import annotations

import numpy as np

import plastax_amd as px
import plastax_amd.numpy as jnp

INCOMING_MARK = -123.5
TRACE = px.FieldSpec.float32("trace", 0.25)
ROLE = px.FieldSpec.float32("role", -1.0)
FWD = px.FieldSpec.float32("fwd")


class LinearForward(px.ForwardPass):
    """Writes its sum to a scratch column, so every unit's ACTIVATION stays
    as built and the update's reads of it have known values."""

    combine = px.monoid.sum_

    def map(self, u, dst, src, c, cid, g):
        return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((FWD, acc))


class OrderProbe(px.UpdateConn):
    def incoming(self, u, dst, src, c, cid, g):
        return px.ConnWrite.of((px.WEIGHT, jnp.float32(INCOMING_MARK)))

    def outgoing(self, u, src, dst, c, cid, g):
        return px.ConnWrite.of((px.WEIGHT, c[px.WEIGHT, cid] + jnp.float32(1000.0)))


class IncomingEndpoint(px.UpdateConn):
    def incoming(self, u, dst, src, c, cid, g):
        return px.ConnWrite.of((px.WEIGHT, u[px.ACTIVATION, dst] - u[px.ACTIVATION, src]))

    def outgoing(self, u, src, dst, c, cid, g):
        return px.ConnWrite.of()


class OutgoingEndpoint(px.UpdateConn):
    def incoming(self, u, dst, src, c, cid, g):
        return px.ConnWrite.of()

    def outgoing(self, u, src, dst, c, cid, g):
        return px.ConnWrite.of((px.WEIGHT, u[px.ACTIVATION, dst] - u[px.ACTIVATION, src]))


class HebbTrace(px.UpdateConn):
    """A nonlinear two-pass rule over two columns: incoming moves the weight
    by a clipped Hebbian term scaled by a global; outgoing decays a
    per-edge trace toward |new weight| and stamps the edge's slot and
    endpoints into ``role`` (cid, src and dst must bind right)."""

    def incoming(self, u, dst, src, c, cid, g):
        hebb = jnp.tanh(u[px.ACTIVATION, dst] * u[px.ACTIVATION, src])
        w = c[px.WEIGHT, cid] + g["lr"] * jnp.clip(hebb, -0.5, 0.5) - jnp.float32(0.01) * c[TRACE, cid]
        return px.ConnWrite.of((px.WEIGHT, w))

    def outgoing(self, u, src, dst, c, cid, g):
        tr = c[TRACE, cid] * jnp.float32(0.5) + jnp.abs(c[px.WEIGHT, cid])
        stamp = (cid * 7 + src * 3 + dst).astype(jnp.float32)
        return px.ConnWrite.of((TRACE, tr), (ROLE, stamp))


def net(rule, propagation=px.Propagation.PIPELINE, extra=()):
    return type("UpdateConnNet", (px.Network,), dict(
        forward_pass=LinearForward(), update_conn=rule, propagation=propagation,
        extra_unit_fields=(FWD,), extra_conn_fields=tuple(extra)))


def endpoint_probe(cls, device: str):
    b = px.NetworkBuilder(net(cls()), None)
    b.add_unit(activation=10.0)
    b.add_unit(activation=20.0)
    b.add_unit(activation=100.0)
    b.add_conn(0, 2, weight=0.0)
    b.add_conn(1, 2, weight=0.0)
    return b.finalize(device=device)


def order_probe_topological(device: str):
    b = px.NetworkBuilder(net(OrderProbe(), px.Propagation.TOPOLOGICAL), None)
    for _ in range(5):
        b.add_unit()
    b.mark_input(0)
    b.mark_input(1)
    b.mark_output(4)
    b.add_conn(0, 2, weight=1.0)
    b.add_conn(1, 2, weight=2.0)
    b.add_conn(2, 3, weight=3.0)
    b.add_conn(3, 4, weight=4.0)
    return b.finalize(device=device)


def random_hebb_net(seed: int, device: str, pipeline: bool):
    rng = np.random.default_rng(seed)
    n = 1200
    if pipeline:
        src = rng.integers(0, n, 9000).astype(np.int32)
        dst = rng.integers(0, n, 9000).astype(np.int32)
        keep = src != dst
        src, dst = src[keep], dst[keep]
        prop = px.Propagation.PIPELINE
    else:
        lv = rng.integers(0, 4, n)
        lv[:40] = 0
        src = rng.integers(0, n, 12000).astype(np.int32)
        dst = rng.integers(0, n, 12000).astype(np.int32)
        keep = lv[src] < lv[dst]
        src, dst = src[keep], dst[keep]
        prop = px.Propagation.TOPOLOGICAL
    w = (rng.standard_normal(src.size) * 0.2).astype(np.float32)
    N = net(HebbTrace(), prop, extra=(TRACE, ROLE))
    static, state = px.NetworkBuilder.from_edges(
        N, n, src, dst, weights=w, input_ids=np.arange(40), output_ids=np.arange(n - 8, n),
        globals_={"lr": np.float32(0.05)}, capacity_headroom=0.5, device=device)
    return N, static, state


class PlainSGD(px.UpdateConn):
    """SGD without the exact batch pair: a batched step takes the mean of
    its per-sample writes (the reference's tests/test_batched.py _PlainSGD)."""

    def __init__(self, lr: float, grad_field) -> None:
        self.lr = np.float32(lr)
        self.grad_field = grad_field

    def incoming(self, u, dst, src, c, cid, g):
        grad = u[self.grad_field, dst] * u[px.ACTIVATION, src]
        return px.ConnWrite.of((px.WEIGHT, c[px.WEIGHT, cid] - self.lr * grad))

    def outgoing(self, u, src, dst, c, cid, g):
        return px.ConnWrite.of()
