"""BASELINE config C5's recipe at 1/32 of its size, 200 steps, against the
oracle: a growing PIPELINE reservoir with per-unit proposals (P = 4) every
step, an out-degree count pass, PruneUnit of zero out-degree units and AddUnit
spawning 16 units every 20 steps. Flags every step; every unit and connection
column (hence compaction, claims and commit order) every 25 steps."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import c5_recipe as c5
import nets
import plastax_amd as px
from test_gpu_parity import assert_same_state

pytestmark = pytest.mark.gpu


def test_c5_recipe_200_steps_bit_exact(oracle) -> None:
    n, cap, n_in = 2048, 8192, 32
    net = c5.recipe(n_in, n, 256, 16, 8, cap)
    src, dst, w = c5.reservoir_edges(0, n, 128 * 1024, n_in)
    static, state = px.NetworkBuilder.from_edges(
        net, n, src, dst, weights=w, input_ids=np.arange(n_in), output_ids=np.arange(n - 8, n),
        globals_={"spawn": np.float32(0.0)}, capacity_headroom=1.0, device="cuda")
    o = nets.oracle_for(oracle, net, static, state)
    o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
    step = px.make_step(net, static)
    assert step.backward_order == "slot"
    o.tile = None
    rng = np.random.default_rng(1)
    added = pruned = 0
    for k in range(1, 201):
        g = {"spawn": np.float32(1.0 if k % 20 == 0 else 0.0)}
        state.globals_, o.globals_ = g, g
        x = rng.standard_normal(n_in).astype(np.float32)
        res = step(state, px.StepInputs(x, None))
        state = res.state
        live_before = int((o.units["pruned"] == 0).sum())
        o.step(x)
        pruned += max(0, live_before - int((o.units["pruned"] == 0).sum()) + o.units_added)
        assert (state.units_added, state.unit_overflow, state.grown, state.overflow, state.tail_start) == (
            o.units_added, o.unit_overflow, o.grown, o.overflow, o.tail_start), f"flags at step {k}"
        added += state.units_added
        if k % 25 == 0:
            torch.cuda.synchronize()
            assert_same_state(static, state, o, f"step {k}")
            print(f"C5 recipe step {k}: every column bit-exact ({added} units added, {pruned} pruned)",
                  flush=True)
    assert added >= 16 * 9 and pruned > 0
