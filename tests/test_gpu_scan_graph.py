"""Driver.scan as a captured HIP graph (the reference's device-side chunk
loop, driver.py:170-260): each chunk's first step runs as usual and the
other steps replay one captured graph. Two identical drivers run the same
chunks, one with graph=True and one step by step (graph=False), with eager
steps between the chunks: every chunk's records and every unit and
connection column after it must be equal bit for bit, and equal to the
oracle's -- for Adam (whose step count the graph reads per edge), SGD, and
a PIPELINE net (whose applies write column copies that the graph returns
into the state's own buffers)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import batched_cases as bc
import nets
import plastax_amd as px
from plastax_amd.driver import Driver
from test_gpu_parity import _equal, assert_same_state

pytestmark = pytest.mark.gpu


def _pipeline_net(opt):
    return nets.make_trained_net("PipeScan", nets.TanhForward(), nets.TanhBackward(), opt, px.Propagation.PIPELINE)


def _build(kind: str, seed: int):
    if kind == "pipeline":
        net = _pipeline_net(px.optim.adam(1e-2, nets.GRAD_PRE_ACT))
        rng = np.random.default_rng(seed)
        n = 400
        src = rng.integers(0, n, 3000).astype(np.int32)
        dst = rng.integers(0, n, 3000).astype(np.int32)
        keep = src != dst
        w = (rng.standard_normal(int(keep.sum())) * 0.2).astype(np.float32)
        static, state = px.NetworkBuilder.from_edges(
            net, n, src[keep], dst[keep], weights=w, input_ids=np.arange(16), output_ids=np.arange(n - 6, n),
            globals_=None, device="cuda")
        return net, static, state, 16, 6
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT) if kind == "adam" else px.optim.sgd(0.05, nets.GRAD_PRE_ACT)
    net = bc.tanh_mse_net(opt)
    static, state = bc.build(net, [20, 48, 40, 8], 0.3, skip=0.05, seed=seed, device="cuda")
    return net, static, state, 20, 8


@pytest.mark.parametrize("kind", ["adam", "sgd", "pipeline"])
def test_scan_graph_equals_step_by_step(oracle, kind: str) -> None:
    runs = []
    for graph in (True, False):
        net, static, state, n_in, n_out = _build(kind, 3)
        runs.append((Driver(net, static, state), graph))
    o = nets.oracle_for(oracle, net, static, runs[0][0].state)
    rng = np.random.default_rng(4)
    K = 7
    for chunk in range(3):
        xs = rng.standard_normal((K, n_in)).astype(np.float32)
        ts = np.tanh(rng.standard_normal((K, n_out))).astype(np.float32)
        steps = K if chunk != 1 else K - 2  # a short chunk: records past `steps` are zero
        print(f"scan chunk {chunk} kind={kind} steps={steps}", flush=True)
        recs = []
        for drv, graph in runs:
            recs.append(drv.scan(px.StepInputs(torch.from_numpy(xs).cuda(), torch.from_numpy(ts).cuda()),
                                 steps=steps, graph=graph))
        torch.cuda.synchronize()
        a, b = (r.cpu().numpy().astype(np.float32) for r in recs)
        assert _equal(a, b), f"chunk {chunk}: records differ"
        want = np.zeros(K, np.float32)
        for i in range(steps):
            want[i] = o.step(xs[i], ts[i])
        assert _equal(a, want), f"chunk {chunk}: records differ from the oracle"
        assert_same_state(static, runs[0][0].state, o, f"chunk {chunk} (graph)")
        assert_same_state(static, runs[1][0].state, o, f"chunk {chunk} (step by step)")
        assert runs[0][0].state.step == runs[1][0].state.step
        # eager steps between the replays
        x = rng.standard_normal(n_in).astype(np.float32)
        t = np.tanh(rng.standard_normal(n_out)).astype(np.float32)
        for drv, _ in runs:
            drv.step(px.StepInputs(x, t))
        o.step(x, t)
        torch.cuda.synchronize()
        assert_same_state(static, runs[0][0].state, o, f"after chunk {chunk}'s eager step")


def test_scan_graph_refusals() -> None:
    net, static, state, n_in, n_out = _build("sgd", 5)
    drv = Driver(net, static, state, check_every=2)
    xs = torch.zeros((3, n_in), device="cuda")
    with pytest.raises(ValueError, match="check_every"):
        drv.scan(px.StepInputs(xs, torch.zeros((3, n_out), device="cuda")), graph=True)
