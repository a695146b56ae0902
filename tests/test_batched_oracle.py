"""The batched oracle (oracle/batched.py), pinned without the device:

- a float64 dense-matrix restatement of a batched MLP step (tanh, MSE, SGD
  on the batch-mean gradient, MEAN-reduced unit columns);
- the reference's own batched assertions (tests/test_batched.py:117-186):
  a batch of one is the streaming step, batched SGD is the mean of B
  streaming SGD steps from the same state;
- the batch reductions' arithmetic (phases.py:298-332) on exact values.
"""

from __future__ import annotations

import numpy as np
import pytest

import batched_cases as bc
import nets
import plastax_amd as px
from plastax_amd._plan import compile_plan


def _oracle(ox, net, static, state, batch):
    from oracle import batched as ob

    o = nets.oracle_for(ox, net, static, state)
    return ob.OracleBatch(o, batch), o


def _dense(static, conns, n):
    W = np.zeros((n, n), dtype=np.float64)  # W[dst, src]
    for c in conns:
        live = ~c["dead"].astype(bool)
        np.add.at(W, (c["to_id"][live], c["from_id"][live]), c["weight"][live].astype(np.float64))
    return W


def test_float64_restatement_of_a_batched_sgd_step(oracle) -> None:
    lr = 0.05
    opt = px.optim.sgd(lr, nets.GRAD_PRE_ACT)
    net = bc.tanh_mse_net(opt)
    layers = [12, 20, 16, 6]
    static, state = bc.build(net, layers, 0.4, skip=0.1, seed=3)
    B = 5
    ob, o = _oracle(oracle, net, static, state, B)
    n = static.num_units
    W = _dense(static, o.conns, n)
    xs, ys = bc.data(1, 1, B, layers[0], layers[-1])
    levels = o.units["level"]
    ins = np.asarray(static.input_ids)
    outs = np.asarray(static.output_ids)
    acts, grads, losses = [], [], []
    for b in range(B):
        a = np.zeros(n)
        a[ins] = xs[0, b]
        for lv in range(1, int(levels.max()) + 1):
            m = levels == lv
            a[m] = np.tanh(W[m] @ a)
        diff = a[outs] - ys[0, b]
        losses.append(0.5 * np.sum(diff * diff))
        seed = np.zeros(n)
        seed[outs] = diff
        gpa = np.zeros(n)
        for lv in range(int(levels.max()), 0, -1):
            m = (levels == lv) & ~np.isin(np.arange(n), ins)
            gpa[m] = (W[:, m].T @ gpa + seed[m]) * (1 - a[m] ** 2)
        acts.append(a)
        grads.append(gpa)
    mean_grad_w = np.mean([np.outer(g, a) for g, a in zip(grads, acts)], axis=0)  # [dst, src]
    W_new = W - lr * mean_grad_w * (W != 0)
    loss = ob.step(xs[0], ys[0])
    np.testing.assert_allclose(float(loss), np.mean(losses), rtol=1e-5)
    got = _dense(static, o.conns, n)
    np.testing.assert_allclose(got, W_new, rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(o.units["activation"], np.mean(acts, axis=0), rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(o.units["grad_pre_act"], np.mean(grads, axis=0), rtol=2e-4, atol=2e-6)


@pytest.mark.parametrize("make", [lambda: px.optim.sgd(0.2, nets.GRAD_PRE_ACT),
                                  lambda: px.optim.adam(0.01, nets.GRAD_PRE_ACT)])
def test_a_batch_of_one_is_the_streaming_step(oracle, make) -> None:
    """tests/test_batched.py:117-135."""
    opt = make()
    net = bc.tanh_mse_net(opt)
    static, state = bc.build(net, [6, 5, 3], 1.0, seed=0)
    ob, o1 = _oracle(oracle, net, static, state, 1)
    o2 = nets.oracle_for(oracle, net, static, state)
    xs, ys = bc.data(1, 5, 1, 6, 3)
    for x, y in zip(xs, ys):
        l1 = ob.step(x, y)
        l2 = o2.step(x[0], y[0])
        np.testing.assert_allclose(float(l1), float(l2), rtol=1e-6, atol=1e-7)
    w1 = np.concatenate([c["weight"] for c in o1.conns])
    w2 = np.concatenate([c["weight"] for c in o2.conns])
    np.testing.assert_allclose(w1, w2, rtol=1e-6, atol=1e-7)


def test_batched_sgd_is_the_mean_of_per_sample_sgd_steps(oracle) -> None:
    """tests/test_batched.py:153-173."""
    opt = px.optim.sgd(0.2, nets.GRAD_PRE_ACT)
    net = bc.tanh_mse_net(opt)
    static, state = bc.build(net, [6, 5, 3], 1.0, seed=0)
    xs, ys = bc.data(2, 1, 4, 6, 3)
    singles = []
    for b in range(4):
        o = nets.oracle_for(oracle, net, static, state)
        o.step(xs[0, b], ys[0, b])
        singles.append(np.concatenate([c["weight"] for c in o.conns]))
    ob, o = _oracle(oracle, net, static, state, 4)
    ob.step(xs[0], ys[0])
    got = np.concatenate([c["weight"] for c in o.conns])
    np.testing.assert_allclose(got, np.mean(singles, axis=0), rtol=1e-5, atol=1e-6)


def test_reductions_are_the_samples_in_order() -> None:
    from oracle import batched as ob

    cols = [np.float32([0.1, 1.0, -0.0, 0.7]), np.float32([0.1, 2.0, -0.0, 0.3]),
            np.float32([0.1, 4.0, -0.0, 0.1])]
    mean = ob.reduce_column("mean", cols, 3)
    want = ((cols[0] + cols[1]) + cols[2]) / np.float32(3)
    assert mean.tobytes() == want.tobytes()
    assert np.signbit(mean[2])  # sums start from sample 0: -0.0 stays -0.0
    assert mean[1] == np.float32(7.0 / 3.0)
    ints = [np.int32([2**31 - 1, 5]), np.int32([1, -7])]
    assert ob.reduce_column("sum", ints, 2).tolist() == [-(2**31), -2]
    assert ob.reduce_column("first", ints, 2).tolist() == [2**31 - 1, 5]


def test_written_columns_are_the_per_sample_outputs() -> None:
    from oracle import batched as ob

    net = bc.tanh_mse_net(px.optim.sgd(0.1, nets.GRAD_PRE_ACT))
    static, _ = bc.build(net, [4, 3, 2], 1.0)
    plan = compile_plan(net, static)
    assert set(ob.written_columns(plan)) == {"activation", "loss_grad", "grad_pre_act"}
