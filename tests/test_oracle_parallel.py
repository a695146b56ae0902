"""The oracle's parallel form (rows / source runs on the OpenMP team, the CPU
baseline's all-core leg) computes the same bits as its sequential form, at
any thread count: every fold keeps its order inside one loop iteration."""

from __future__ import annotations

import numpy as np
import pytest

import nets
import plastax_amd as px
from plastax_amd import synth


@pytest.mark.parametrize("rule", ["adam", "sgd"])
def test_parallel_oracle_matches_sequential_bit_for_bit(oracle, rule: str) -> None:
    e = synth.c2_topological(seed=3, scale=64, layers=4)  # 2,048-wide Zipf layers: the loops run parallel
    opt = px.optim.adam(1e-3, nets.GRAD_PRE_ACT) if rule == "adam" else px.optim.sgd(1e-2, nets.GRAD_PRE_ACT)
    net = nets.make_trained_net("P", nets.TanhForward(), nets.TanhBackward(), opt, px.Propagation.TOPOLOGICAL)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cpu")
    rng = np.random.default_rng(0)
    xs = rng.standard_normal((4, e.input_ids.size)).astype(np.float32)
    ts = np.tanh(xs[:, ::-1]).astype(np.float32)
    runs = []
    for parallel, threads in ((False, 1), (True, 1), (True, 4)):
        o = nets.oracle_for(oracle, net, static, state, parallel=parallel)
        o.lib.ox_set_threads(threads)
        losses = [o.step(x, t) for x, t in zip(xs, ts)]
        runs.append((losses, o.units, o.conns))
    o.lib.ox_set_threads(1)
    ref_l, ref_u, ref_c = runs[0]
    for losses, units, conns in runs[1:]:
        assert [np.float32(v).view(np.uint32) for v in losses] == [np.float32(v).view(np.uint32) for v in ref_l]
        for k, v in ref_u.items():
            assert np.array_equal(units[k].view(np.uint8), v.view(np.uint8)), k
        for b, bucket in enumerate(ref_c):
            for k, v in bucket.items():
                assert np.array_equal(conns[b][k].view(np.uint8), v.view(np.uint8)), (b, k)
