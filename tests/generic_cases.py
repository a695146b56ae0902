"""Nets whose passes are outside the product form (plastax_amd/generic.py),
after the reference's examples: a nonlinear map (ipc_multilayer.py's
``w * f(x[src])``), a tuple accumulator with a tuple of monoids (xmc.py's
``(1, |w|)``, upgd.py's ``(weighted, util)`` under (sum, max)), a backward
map of three factors. Shared by the oracle tests and the device tests."""

from __future__ import annotations

import numpy as np

import nets
import plastax_amd as px
import plastax_amd.numpy as jnp

UTIL = px.FieldSpec.float32("test/util", 0.5)
DEG = px.FieldSpec.float32("test/deg")
MX = px.FieldSpec.float32("test/mx")
MN = px.FieldSpec.float32("test/mn")
PR = px.FieldSpec.float32("test/pr")


class TanhSrcForward(px.ForwardPass):
    """Nonlinear map: the source's activation squashed again."""

    combine = px.monoid.sum_

    def map(self, u, dst, src, c, cid, g):
        return c[px.WEIGHT, cid] * jnp.tanh(u[px.ACTIVATION, src])

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)))


class TupleForward(px.ForwardPass):
    """(weighted input, max |w| * util) under (sum, max), and the in-degree."""

    combine = (px.monoid.sum_, px.monoid.max_, px.monoid.sum_)

    def map(self, u, dst, src, c, cid, g):
        return (c[px.WEIGHT, cid] * u[px.ACTIVATION, src], jnp.abs(c[px.WEIGHT, cid]) * c[UTIL, cid],
                jnp.float32(1.0))

    def apply(self, u, i, g, acc):
        s, m, n = acc
        return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(s) + m * jnp.float32(0.01)), (DEG, n), (MX, m))


class MinProdMaxForward(px.ForwardPass):
    """(min util, product of util, max |w| * util) under (min, prod, max):
    every named monoid but sum in one tuple; each component is also written
    to its own unit column."""

    combine = (px.monoid.min_, px.monoid.prod, px.monoid.max_)

    def map(self, u, dst, src, c, cid, g):
        return (c[UTIL, cid], c[UTIL, cid], jnp.abs(c[px.WEIGHT, cid]) * c[UTIL, cid])

    def apply(self, u, i, g, acc):
        mn, pr, mx = acc
        return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(mn + pr * jnp.float32(0.01))), (MN, mn), (PR, pr),
                               (MX, mx))


class ProductAsTupleForward(px.ForwardPass):
    """The product map written as a one-element tuple: runs as a generic pass
    and must give the product path's bits."""

    combine = (px.monoid.sum_,)

    def map(self, u, dst, src, c, cid, g):
        return (c[px.WEIGHT, cid] * u[px.ACTIVATION, src],)

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc[0])))


class ThreeFactorBackward(px.BackwardPass):
    """w * g[dst] * (1 + act[src]^2): outside the product form."""

    combine = px.monoid.sum_

    def map(self, u, src, dst, c, cid, g):
        a = u[px.ACTIVATION, src]
        return c[px.WEIGHT, cid] * u[nets.GRAD_PRE_ACT, dst] * (jnp.float32(1.0) + a * a)

    def apply(self, u, i, g, acc):
        a = u[px.ACTIVATION, i]
        return px.UnitWrite.of((nets.GRAD_PRE_ACT, (acc + u[nets.LOSS_GRAD, i]) * (jnp.float32(1.0) - a * a)))


class ProductAsTupleBackward(px.BackwardPass):
    combine = (px.monoid.sum_,)

    def map(self, u, src, dst, c, cid, g):
        return (c[px.WEIGHT, cid] * u[nets.GRAD_PRE_ACT, dst],)

    def apply(self, u, i, g, acc):
        a = u[px.ACTIVATION, i]
        return px.UnitWrite.of((nets.GRAD_PRE_ACT, (acc[0] + u[nets.LOSS_GRAD, i]) * (jnp.float32(1.0) - a * a)))


def make_net(forward, backward, *, pipeline: bool = False, optimizer=None):
    opt = optimizer or px.optim.sgd(0.05, nets.GRAD_PRE_ACT)

    class Net(px.Network):
        forward_pass = forward
        backward_pass = backward
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD, DEG, MX, MN, PR)
        extra_conn_fields = (UTIL, *tuple(opt.state_fields))
        propagation = px.Propagation.PIPELINE if pipeline else px.Propagation.TOPOLOGICAL

    return Net


def build(net, *, pipeline: bool, seed: int, device: str = "cpu"):
    rng = np.random.default_rng(seed)
    if pipeline:
        n = 300
        src = rng.integers(0, n, 1800).astype(np.int32)
        dst = rng.integers(0, n, 1800).astype(np.int32)
        keep = src != dst
        src, dst = src[keep], dst[keep]
        ins, outs = np.arange(16), np.arange(n - 8, n)
    else:
        layers = [24, 60, 50, 8]
        base = np.concatenate([[0], np.cumsum(layers)])
        src, dst = [], []
        for l in range(len(layers) - 1):
            a = np.arange(base[l], base[l + 1])
            b = np.arange(base[l + 1], base[l + 2])
            m = rng.random((a.size, b.size)) < 0.3
            ii, jj = np.nonzero(m)
            src.append(a[ii])
            dst.append(b[jj])
        # a few skip edges (rows carried across buckets)
        src.append(rng.integers(0, layers[0], 30))
        dst.append(rng.integers(base[2], base[3], 30))
        src = np.concatenate(src).astype(np.int32)
        dst = np.concatenate(dst).astype(np.int32)
        n = int(base[-1])
        ins, outs = np.arange(layers[0]), np.arange(base[-2], base[-1])
    w = (rng.standard_normal(src.size) * 0.3).astype(np.float32)
    return px.NetworkBuilder.from_edges(net, n, src, dst, weights=w, input_ids=ins, output_ids=outs,
                                        globals_=None, capacity_headroom=0.25, device=device)


def data(seed: int, steps: int, n_in: int, n_out: int) -> tuple[np.ndarray, np.ndarray]:
    rng = np.random.default_rng(seed)
    xs = rng.standard_normal((steps, n_in)).astype(np.float32)
    ts = np.tanh(rng.standard_normal((steps, n_out))).astype(np.float32)
    return xs, ts
