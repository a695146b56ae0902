"""C4 at its full shape: dynamic sparse training, device vs oracle, bit for bit.

C3's sparse MLP (784-4096-4096-10, each dense layer pair's edge kept w.p.
0.1: 2,004,393 edges) at batch 1, tanh units (their gradients stay alive, so
the regrowth scores are not all zero), softmax cross-entropy, Adam(1e-3).
Every 100 steps (steps 1 and 101):

- PruneConn drops the live edges whose |w| is below g["tau"], the 10th
  percentile of the live |w| before the step (set in the globals from the
  oracle's arrays, so both sides prune with the same threshold);
- ScoreAddConn regrows from a 32 x 32 shortlist per level (1,024 candidates)
  scored by |act[src] * grad[dst]|, up to 1,024 new edges per level, new
  weights 0, live pairs deduplicated.

The structural flags agree at every step; every unit column, every logical
connection column (so the compaction and the commit order) and the loss agree
at the checked steps.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import nets
import plastax_amd as px
import plastax_amd.numpy as jnp
from plastax_amd import synth
from test_gpu_parity import _equal, assert_same_state

pytestmark = pytest.mark.gpu


class C4Prune(px.PruneConn):
    def predicate(self, u, c, cid, g):
        return jnp.abs(c[px.WEIGHT, cid]) < g["tau"]


class C4Grow(px.ScoreAddConn):
    candidates = "shortlist_per_level"
    shortlist_size = 32
    direction = "deeper"
    max_level_gap = 1
    dedupe_live = True
    max_new_per_level = 1024
    trigger = ("every", 100)

    def score(self, u, src, dst, g):
        return jnp.abs(u[px.ACTIVATION, src] * u[nets.GRAD_PRE_ACT, dst])

    def importance(self, u, i, g):
        return jnp.abs(u[nets.GRAD_PRE_ACT, i]) + jnp.abs(u[px.ACTIVATION, i])

    def init(self, u, src, dst, g):
        return px.ConnWrite.of((px.WEIGHT, jnp.float32(0.0)))


def _live_abs_weight_quantile(o, q: float) -> np.float32:
    w = np.concatenate([np.abs(c["weight"][~c["dead"].astype(bool)]) for c in o.conns])
    return np.float32(np.quantile(w, q))


def test_c4_dynamic_sparse_training_full_shape_bit_exact(oracle) -> None:
    e = synth.c3_mlp(seed=0)
    opt = px.optim.adam(1e-3, nets.GRAD_PRE_ACT)

    class C4(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = px.SoftmaxCrossEntropyLoss(nets.LOSS_GRAD)
        update_conn = opt.update_conn()
        prune_conn = C4Prune()
        add_conn = C4Grow()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        extra_conn_fields = tuple(opt.state_fields)

    static, state = px.NetworkBuilder.from_edges(
        C4, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids, output_ids=e.output_ids,
        globals_={"tau": np.float32(0.0)}, capacity_headroom=0.1, device="cuda")
    o = nets.oracle_for(oracle, C4, static, state)
    o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
    step = px.make_step(C4, static)
    if step.backward_order == "slot":
        o.tile = None
    steps = 101
    xs, ys = synth.c3_batches(0, steps, 1)
    check_at = {1, 2, 50, 100, 101}
    grown = pruned = 0
    for k in range(1, steps + 1):
        tau = _live_abs_weight_quantile(o, 0.1) if (k - 1) % 100 == 0 else np.float32(0.0)
        state.globals_ = {"tau": tau}
        o.globals_ = {"tau": tau}
        live_before = sum(int((c["dead"] == 0).sum()) for c in o.conns)
        x, t = xs[k - 1, 0], ys[k - 1, 0]
        res = step(state, px.StepInputs(x, t))
        state = res.state
        lo = o.step(x, t)
        assert (state.grown, state.overflow, state.needs_resort, state.tail_start) == (
            o.grown, o.overflow, o.needs_resort, o.tail_start), f"flags at step {k}"
        grown += state.grown
        if tau > 0:
            pruned += live_before + state.grown - sum(int((c["dead"] == 0).sum()) for c in o.conns)
        if k in check_at:
            print(f"C4 step {k}: checking", flush=True)
            torch.cuda.synchronize()
            assert_same_state(static, state, o, f"step {k}")
            assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at {k}"
    # two prune + regrow events: about 10 % of the live edges pruned each time, and
    # up to 1,024 edges regrown per level
    assert pruned > 2 * 150_000 and grown > 2 * 1024


def test_c4_eleven_prune_and_regrow_events_bit_exact(oracle) -> None:
    """C4 for 1,001 steps: eleven prune + regrow events (steps 1, 101, ...,
    1001), against the oracle's parallel form (the same folds, OpenMP on the
    host's cores). The flags at every step; every unit and connection column
    and the loss after each event's step and at the end."""
    import os
    import time

    e = synth.c3_mlp(seed=0)
    opt = px.optim.adam(1e-3, nets.GRAD_PRE_ACT)

    class C4(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = px.SoftmaxCrossEntropyLoss(nets.LOSS_GRAD)
        update_conn = opt.update_conn()
        prune_conn = C4Prune()
        add_conn = C4Grow()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        extra_conn_fields = tuple(opt.state_fields)

    static, state = px.NetworkBuilder.from_edges(
        C4, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids, output_ids=e.output_ids,
        globals_={"tau": np.float32(0.0)}, capacity_headroom=0.1, device="cuda")
    o = nets.oracle_for(oracle, C4, static, state, parallel=True)
    o.lib.ox_set_threads(min(16, len(os.sched_getaffinity(0))))
    o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
    step = px.make_step(C4, static)
    if step.backward_order == "slot":
        o.tile = None
    steps = 1001
    xs, ys = synth.c3_batches(1, steps, 1)
    check_at = {1, 2, 101, 102, 501, 502, 1001}
    events = grown = 0
    t0 = time.perf_counter()
    try:
        for k in range(1, steps + 1):
            prune = (k - 1) % 100 == 0
            tau = _live_abs_weight_quantile(o, 0.1) if prune else np.float32(0.0)
            state.globals_ = {"tau": tau}
            o.globals_ = {"tau": tau}
            x, t = xs[k - 1, 0], ys[k - 1, 0]
            res = step(state, px.StepInputs(x, t))
            state = res.state
            lo = o.step(x, t)
            assert (state.grown, state.overflow, state.needs_resort, state.tail_start) == (
                o.grown, o.overflow, o.needs_resort, o.tail_start), f"flags at step {k}"
            grown += state.grown
            events += int(prune and state.grown > 0)
            if k in check_at:
                torch.cuda.synchronize()
                assert_same_state(static, state, o, f"step {k}")
                assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at {k}"
                print(f"[{time.perf_counter() - t0:6.1f} s] C4 step {k}: every column bit-exact", flush=True)
    finally:
        o.lib.ox_set_threads(1)
    assert events == 11 and grown > 11 * 1024
