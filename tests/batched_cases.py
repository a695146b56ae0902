"""Batched-step nets for the oracle and device tests (make_step(batch_size=B),
step.py:359-468): sparse layered MLPs with optional skip edges, trained with
an optim bundle on the batch-mean gradient."""

from __future__ import annotations

import numpy as np

import nets
import plastax_amd as px


def sparse_mlp(rng: np.random.Generator, layers: list[int], keep: float, skip: float = 0.0):
    """(n, src, dst, w, input_ids, output_ids) of a layered net, each layer
    pair kept with probability `keep`, plus skip edges two layers up with
    probability `skip`; weights N(0, 1/fan_in)."""
    base = np.concatenate([[0], np.cumsum(layers)])
    src, dst = [], []
    for l in range(len(layers) - 1):
        for up, p in ((1, keep), (2, skip)):
            if l + up >= len(layers) or p <= 0:
                continue
            a = np.arange(base[l], base[l + 1])
            b = np.arange(base[l + up], base[l + up + 1])
            m = rng.random((a.size, b.size)) < p
            ii, jj = np.nonzero(m)
            src.append(a[ii])
            dst.append(b[jj])
    src = np.concatenate(src).astype(np.int32)
    dst = np.concatenate(dst).astype(np.int32)
    fan = np.bincount(dst, minlength=int(base[-1]))
    w = (rng.standard_normal(src.size) / np.sqrt(np.maximum(fan[dst], 1))).astype(np.float32)
    return int(base[-1]), src, dst, w, np.arange(layers[0]), np.arange(base[-2], base[-1])


def tanh_mse_net(opt):
    class Net(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        extra_conn_fields = tuple(opt.state_fields)
        batch_reduction = px.MeanFloatFirstRest()

    return Net


def softmax_net(opt):
    class Net(px.Network):
        forward_pass = nets.ReluForward()
        backward_pass = nets.ReluBackward()
        loss = px.SoftmaxCrossEntropyLoss(nets.LOSS_GRAD)
        update_conn = opt.update_conn()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        extra_conn_fields = tuple(opt.state_fields)
        batch_reduction = px.MeanFloatFirstRest()

    return Net


def build(net, layers, keep, skip=0.0, seed=0, device="cpu", headroom=0.0):
    rng = np.random.default_rng(seed)
    n, src, dst, w, ins, outs = sparse_mlp(rng, layers, keep, skip)
    return px.NetworkBuilder.from_edges(net, n, src, dst, weights=w, input_ids=ins, output_ids=outs,
                                        globals_=None, capacity_headroom=headroom, device=device)


def data(seed: int, steps: int, batch: int, n_in: int, n_out: int, onehot: bool = False):
    rng = np.random.default_rng(seed)
    xs = rng.standard_normal((steps, batch, n_in)).astype(np.float32)
    if onehot:
        lab = rng.integers(0, n_out, (steps, batch))
        ys = np.eye(n_out, dtype=np.float32)[lab]
    else:
        ys = (rng.standard_normal((steps, batch, n_out)) * 0.5).astype(np.float32)
    return xs, ys
