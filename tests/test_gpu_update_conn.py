"""User UpdateConn policies on the device (edge programs on the physical
arena): the reference's known answers (tests/test_update_conn.py) and
nonlinear two-pass rules against the oracle bit for bit, in both
propagation modes, with tombstones inside the live range and in the churn
layout."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import nets
import plastax_amd as px
import plastax_amd.numpy as jnp
import update_conn_cases as uc
from test_gpu_parity import assert_same_state

pytestmark = pytest.mark.gpu


def _step(net, static, state, k=1):
    step = px.make_step(net, static)
    for _ in range(k):
        state = step(state, px.StepInputs(np.zeros(len(static.input_ids), np.float32))).state
    torch.cuda.synchronize()
    return state


def test_endpoint_probes_on_the_device() -> None:
    for cls in (uc.IncomingEndpoint, uc.OutgoingEndpoint):
        static, state = uc.endpoint_probe(cls, "cuda")
        state = _step(uc.net(cls()), static, state)
        w = state.conns[0]["weight"].cpu().numpy()
        dead = state.conns[0]["dead"].cpu().numpy().astype(bool)
        assert sorted(w[~dead].tolist()) == [80.0, 90.0]


def test_order_probe_in_every_bucket_on_the_device() -> None:
    static, state = uc.order_probe_topological("cuda")
    state = _step(uc.net(uc.OrderProbe(), px.Propagation.TOPOLOGICAL), static, state)
    for bucket in state.conns:
        w = bucket["weight"].cpu().numpy()
        dead = bucket["dead"].cpu().numpy().astype(bool)
        assert (w[~dead] == np.float32(uc.INCOMING_MARK + 1000.0)).all()
        assert (w[dead] == 0.0).all()


class TauPrune(px.PruneConn):
    def predicate(self, u, c, cid, g):
        return jnp.abs(c[px.WEIGHT, cid]) < g["tau"]


class Propose(px.ProposeAddConn):
    proposer = "per_unit"
    proposals_per_proposer = 2
    max_new_per_level = 6
    max_level_gap = 1 << 20

    def propose(self, u, i, j, g, rng):
        return jnp.asarray(i, jnp.int32), rng.uniform_int(1200).astype(jnp.int32), rng.uniform()

    def init(self, u, src, dst, g):
        return px.ConnWrite.of((px.WEIGHT, jnp.float32(0.05)), (uc.TRACE, jnp.float32(0.5)))


@pytest.mark.parametrize("pipeline,prune,grow", [(True, False, False), (False, False, False),
                                                 (False, True, False), (True, True, True)])
def test_hebb_trace_rule_matches_oracle(oracle, pipeline: bool, prune: bool, grow: bool) -> None:
    net, static, state = uc.random_hebb_net(3, "cuda", pipeline)
    if prune or grow:
        extra = {}
        if prune:
            extra["prune_conn"] = TauPrune()
        if grow:
            extra["add_conn"] = Propose()
        net = type("HebbPlus", (net,), extra)
        src, dst, w = _edges(state)
        static, state = px.NetworkBuilder.from_edges(
            net, static.num_units, src, dst, weights=w, input_ids=list(static.input_ids),
            output_ids=list(static.output_ids), globals_={"lr": np.float32(0.05), "tau": np.float32(0.0)},
            capacity_headroom=0.5, device="cuda")
    o = nets.oracle_for(oracle, net, static, state)
    o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
    step = px.make_step(net, static)
    if step.backward_order == "slot":
        o.tile = None
    rng = np.random.default_rng(8)
    for k in range(1, 7):
        g = {"lr": np.float32(0.05 * k), "tau": np.float32(0.02 * (k % 2))}
        state.globals_, o.globals_ = g, g
        x = rng.standard_normal(len(static.input_ids)).astype(np.float32)
        print(f"hebb step {k} pipeline={pipeline} prune={prune} grow={grow}", flush=True)
        state = step(state, px.StepInputs(x)).state
        o.step(x)
        torch.cuda.synchronize()
        assert_same_state(static, state, o, f"step {k}")


def _edges(state):
    src, dst, w = [], [], []
    for b in state.conns:
        live = b["dead"].cpu().numpy() == 0
        src.append(b["from_id"].cpu().numpy()[live])
        dst.append(b["to_id"].cpu().numpy()[live])
        w.append(b["weight"].cpu().numpy()[live])
    return np.concatenate(src), np.concatenate(dst), np.concatenate(w)
