"""Losses beyond MSE / softmax CE on the device (k_loss_pieces with log1p,
exp, abs, sigmoid; a loss reading one fixed unit through plx_program's
fixed_mask): bit-exact with the oracle over training steps, streaming and
batched."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import batched_cases as bc
import loss_cases as lc
import nets
import plastax_amd as px
from test_gpu_parity import _equal, assert_same_state

pytestmark = pytest.mark.gpu

LOSSES = [lc.WeightedLogisticLoss(2.5), lc.TdLoss(3), lc.TdLoss(lc.LAYERS[0] + 5)]


@pytest.mark.parametrize("loss", LOSSES, ids=["logistic", "td_input_unit", "td_hidden_unit"])
def test_streaming_losses_match_the_oracle(oracle, loss) -> None:
    net = lc.make_net(loss)
    static, state = lc.build(net, seed=4, device="cuda")
    o = nets.oracle_for(oracle, net, static, state)
    step = px.make_step(net, static)
    rng = np.random.default_rng(5)
    for k in range(6):
        print(f"loss step {k} {type(loss).__name__}", flush=True)
        x = rng.standard_normal(len(static.input_ids)).astype(np.float32)
        t = lc.targets_for(loss, rng, len(static.output_ids))
        res = step(state, px.StepInputs(x, t))
        state = res.state
        lo = o.step(x, t)
        torch.cuda.synchronize()
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at step {k}"
        assert_same_state(static, state, o, f"step {k}")


@pytest.mark.parametrize("loss", LOSSES[:2], ids=["logistic", "td_input_unit"])
@pytest.mark.parametrize("B", [4, 16])
def test_batched_losses_match_the_oracle(oracle, loss, B: int) -> None:
    from oracle import batched as ob

    net = lc.make_net(loss, batched=True)
    static, state = lc.build(net, seed=6, device="cuda")
    o = nets.oracle_for(oracle, net, static, state)
    o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
    orc = ob.OracleBatch(o, B)
    step = px.make_step(net, static, batch_size=B)
    rng = np.random.default_rng(7)
    for k in range(3):
        print(f"batched loss step {k} {type(loss).__name__} B={B}", flush=True)
        x = rng.standard_normal((B, len(static.input_ids))).astype(np.float32)
        t = lc.targets_for(loss, rng, (B, len(static.output_ids)))
        res = step(state, px.StepInputs(x, t))
        state = res.state
        lo = orc.step(x, t)
        torch.cuda.synchronize()
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at step {k}"
        assert_same_state(static, state, o, f"step {k}")
