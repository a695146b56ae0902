"""Pins of the oracle's step arithmetic by closed forms and brute force.

- Optimizer rules on single edges with values whose float32 arithmetic is
  exact (dyadic), or against their closed forms (Adam's bias correction
  makes a constant-gradient step exactly lr * g / (|g| + eps) in real
  arithmetic).
- Forward / backward / update of random topological and pipeline nets
  against an independent float64 dense-matrix restatement, to rel 1e-5:
  a dropped term, a transposed operand or a wrong level order fails it.
"""

from __future__ import annotations

import numpy as np
import pytest

import nets
import plastax_amd as px


def _sum_map(field: str):
    """The linear sum_ map over ``field`` as the oracle's pass plans state it."""
    import types

    return types.SimpleNamespace(field=field, monoid=0, w_const=None, x_const=None)


def _single_edge_net(opt):
    return nets.make_trained_net(
        "One_" + type(opt).__name__, nets.LinearForward(), nets.TanhBackward(), opt,
        px.Propagation.TOPOLOGICAL,
    )


def _one_edge(oracle, opt, w0: float, act_src: float, grad_dst: float):
    """An OracleNet with a single live edge 0 -> 1 whose update sees
    activation[0] = act_src and grad_pre_act[1] = grad_dst."""
    net = _single_edge_net(opt)
    static, state = px.NetworkBuilder.from_edges(
        net, 2, np.int32([0]), np.int32([1]), weights=np.float32([w0]),
        input_ids=[0], output_ids=[1], globals_=None, device="cpu")
    o = nets.oracle_for(oracle, net, static, state)
    o.units["activation"][0] = act_src
    o.units["grad_pre_act"][1] = grad_dst
    return o


def test_sgd_step_exact(oracle) -> None:
    o = _one_edge(oracle, px.optim.sgd(0.125, nets.GRAD_PRE_ACT), 0.5, 2.0, 0.25)
    o.update()
    assert o.conns[0]["weight"][0] == np.float32(0.5 - 0.125 * 0.5)


def test_momentum_two_steps_exact(oracle) -> None:
    o = _one_edge(oracle, px.optim.momentum(0.25, 0.5, nets.GRAD_PRE_ACT), 1.0, 1.0, 0.25)
    o.update()
    o.update()
    # v1 = g, v2 = mu*g + g; w2 = w0 - lr*v1 - lr*v2
    assert o.conns[0]["opt/v"][0] == np.float32(0.375)
    assert o.conns[0]["weight"][0] == np.float32(1.0 - 0.25 * 0.25 - 0.25 * 0.375)


@pytest.mark.parametrize("g", [0.3, -1.7, 1e-3])
def test_adam_constant_gradient_moves_lr_per_step(oracle, g: float) -> None:
    """With a constant gradient, m_hat = g and v_hat = g^2 exactly in real
    arithmetic for every t (the bias corrections cancel 1 - b^t), so each
    step moves w by lr * g / (|g| + eps)."""
    lr, eps = 1e-3, 1e-8
    o = _one_edge(oracle, px.optim.adam(lr, nets.GRAD_PRE_ACT), 0.0, 1.0, g)
    for t in range(1, 201):
        o.update()
        want = -t * lr * g / (abs(g) + eps)
        assert abs(o.conns[0]["weight"][0] - want) <= 1e-5 * abs(want) + 1e-7, t
    assert o.conns[0]["opt/t"][0] == 200.0


def test_adamw_decay_with_zero_gradient(oracle) -> None:
    """g = 0 leaves m = v = 0, so the step is the decoupled decay alone."""
    lr, wd = 0.5, 0.25
    o = _one_edge(oracle, px.optim.adamw(lr, nets.GRAD_PRE_ACT, weight_decay=wd), 2.0, 1.0, 0.0)
    o.update()
    assert o.conns[0]["weight"][0] == np.float32(2.0 - lr * wd * 2.0)


def test_rmsprop_first_step_closed_form(oracle) -> None:
    lr, d, eps, g = 1e-2, 0.9, 1e-8, 0.5
    o = _one_edge(oracle, px.optim.rmsprop(lr, nets.GRAD_PRE_ACT, decay=d, eps=eps), 0.0, 1.0, g)
    o.update()
    want = -lr * g / np.sqrt((1 - d) * g * g + eps)
    assert abs(o.conns[0]["weight"][0] - want) <= 2e-7 * abs(want)


# ---------------------------------------------------------------------------
# Whole passes against a float64 dense restatement.
# ---------------------------------------------------------------------------


def _random_dag(rng, layers=(5, 7, 6, 3), density=0.6, skip=True):
    """Layered DAG with optional skip edges; returns src, dst, weight, n."""
    offs = np.concatenate([[0], np.cumsum(layers)])
    src, dst = [], []
    for li in range(1, len(layers)):
        for d in range(offs[li], offs[li + 1]):
            for lj in range(li):
                if lj != li - 1 and not skip:
                    continue
                for s in range(offs[lj], offs[lj + 1]):
                    if rng.random() < (density if lj == li - 1 else 0.2):
                        src.append(s)
                        dst.append(d)
    n = int(offs[-1])
    w = rng.standard_normal(len(src)).astype(np.float32)
    return np.int32(src), np.int32(dst), w, n, layers


def _dense_f64_step(src, dst, w, n, inputs, out_ids, targets, levels):
    """Forward (tanh), MSE and backward in float64 with a dense matrix."""
    W = np.zeros((n, n))
    np.add.at(W, (dst, src), w.astype(np.float64))
    a = np.zeros(n)
    a[: len(inputs)] = inputs
    for lv in range(1, levels.max() + 1):
        idx = np.flatnonzero(levels == lv)
        a[idx] = np.tanh(W[idx] @ a)
    seed = np.zeros(n)
    seed[out_ids] = a[out_ids] - targets
    grad = np.zeros(n)
    for lv in range(levels.max(), 0, -1):
        idx = np.flatnonzero(levels == lv)
        grad[idx] = (W[:, idx].T @ grad + seed[idx]) * (1 - a[idx] ** 2)
    return a, grad


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_topological_pass_matches_float64_dense(oracle, seed: int) -> None:
    rng = np.random.default_rng(seed)
    src, dst, w, n, layers = _random_dag(rng)
    n_in, n_out = layers[0], layers[-1]
    out_ids = list(range(n - n_out, n))
    net = nets.make_trained_net(f"D{seed}", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.sgd(0.0, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state = px.NetworkBuilder.from_edges(
        net, n, src, dst, weights=w, input_ids=list(range(n_in)), output_ids=out_ids,
        globals_=None, device="cpu")
    o = nets.oracle_for(oracle, net, static, state)
    x = rng.standard_normal(n_in).astype(np.float32)
    t = rng.standard_normal(n_out).astype(np.float32)
    loss = o.step(x, t)
    a64, g64 = _dense_f64_step(src, dst, w, n, x, out_ids, t, o.units["level"])
    np.testing.assert_allclose(o.units["activation"], a64, rtol=1e-5, atol=1e-6)
    non_input = np.arange(n) >= n_in
    np.testing.assert_allclose(o.units["grad_pre_act"][non_input], g64[non_input], rtol=1e-5, atol=1e-6)
    want_loss = 0.5 * np.sum((a64[out_ids] - t) ** 2)
    np.testing.assert_allclose(loss, want_loss, rtol=1e-5)


def test_pipeline_pass_matches_float64_dense(oracle) -> None:
    """PIPELINE: every non-input unit reads the previous step's activations;
    backward reads the previous step's grads and applies to every unit."""
    rng = np.random.default_rng(5)
    n, m = 40, 160
    src = rng.integers(0, n, m).astype(np.int32)
    dst = rng.integers(0, n, m).astype(np.int32)
    w = rng.standard_normal(m).astype(np.float32) * 0.3
    n_in, out_ids = 4, [38, 39]
    net = nets.make_trained_net("Pp", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.sgd(0.0, nets.GRAD_PRE_ACT), px.Propagation.PIPELINE)
    static, state = px.NetworkBuilder.from_edges(
        net, n, src, dst, weights=w, input_ids=list(range(n_in)), output_ids=out_ids,
        globals_=None, device="cpu")
    o = nets.oracle_for(oracle, net, static, state)
    W = np.zeros((n, n))
    np.add.at(W, (dst, src), w.astype(np.float64))
    a = np.zeros(n)
    grad = np.zeros(n)
    for _ in range(6):
        x = rng.standard_normal(n_in).astype(np.float32)
        t = rng.standard_normal(2).astype(np.float32)
        o.step(x, t)
        a_prev = a.copy()
        a_prev[:n_in] = x
        a_new = np.tanh(W @ a_prev)
        a_new[:n_in] = x
        seed = np.zeros(n)
        seed[out_ids] = a_new[out_ids] - t
        grad = (W.T @ grad + seed) * (1 - a_new**2)
        a = a_new
        np.testing.assert_allclose(o.units["activation"], a, rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(o.units["grad_pre_act"], grad, rtol=1e-5, atol=1e-6)


def test_backward_pieces_only_regroup_the_slot_order_fold(oracle) -> None:
    """A hub source with 1,000 out-edges: the 256-term pieces change only the
    grouping of the sum, within float32 rounding of the plain fold."""
    n_dst = 1000
    n = 2 + n_dst
    src = np.concatenate([np.zeros(n_dst, np.int32)])
    dst = np.arange(2, n, dtype=np.int32)
    rng = np.random.default_rng(3)
    w = rng.standard_normal(n_dst).astype(np.float32)
    net = nets.make_trained_net("Hub", nets.LinearForward(), nets.TanhBackward(),
                                px.optim.sgd(0.0, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    res = {}
    for piece in (256, 1 << 20):
        static, state = px.NetworkBuilder.from_edges(
            net, n, src, np.int32(dst), weights=w, input_ids=[0, 1],
            output_ids=list(range(2, n)), globals_=None, device="cpu")
        o = nets.oracle_for(oracle, net, static, state, piece=piece)
        o.units["grad_pre_act"][2:] = rng.standard_normal(n_dst).astype(np.float32)
        o.units["level"][:] = 1
        o.units["level"][0] = 1
        out = o._reduce_bwd(0, _sum_map("grad_pre_act"))
        res[piece] = out[0]
        rng = np.random.default_rng(3)
        rng.standard_normal(n_dst)
    exact = float(np.dot(w.astype(np.float64), o.units["grad_pre_act"][2:].astype(np.float64)))
    assert abs(res[256] - exact) <= 1e-5 * max(1.0, abs(exact))
    assert abs(res[1 << 20] - exact) <= 1e-5 * max(1.0, abs(exact))
