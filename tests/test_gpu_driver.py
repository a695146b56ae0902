"""The host Driver on the device against the oracle's Driver, bit for bit:
overflowing growth completed in the same step (grow_bucket + the retry of
the dropped winners), TOPOLOGICAL resorts (levels recomputed, buckets laid
out again), and the device resort and growth retry on their own."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import growth_cases as gc
import nets
import plastax_amd as px
import plastax_amd.numpy as jnp
from oracle import growth as og
from plastax_amd import grow
from plastax_amd.driver import Driver
from plastax_amd.resort import resort as device_resort
from plastax_amd.state import NetworkState, column_to_numpy, to_column
from test_gpu_growth import _same_arena, _to_device, _to_host
from test_gpu_parity import _equal, assert_same_state

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def test_growth_retry_golden_on_device() -> None:
    """grow_claim_topological_regrow: the attempt, the Driver's regrow, the
    retry of the dropped winners (test_parity_goldens.py:863-930)."""
    doc = gc.load("grow_claim_topological_regrow")
    free = {int(k): v for k, v in doc["params"]["free_per_level"].items()}
    hn = gc.score_net(doc, step_cap=None, free_at=free)
    units, conns = _to_device(hn)
    phase = grow.AddConnPhase(hn.net, hn.static, hn.globals_)
    k = grow.Kernels(DEV, torch.cuda.current_stream(DEV).cuda_stream)
    out = phase.run(k, units, conns, step=hn.step, globals_=hn.globals_)
    attempt = _to_host(hn, out.conns)
    assert gc.grown_pairs(hn.conns, attempt) == gc.want_commits(doc["expect"])
    full = [b for b, c in enumerate(attempt) if not c["dead"].any()]
    static, hconns = hn.static, attempt
    for lvl in full:
        static, hconns = og.grow_bucket(static, hconns, lvl)
    retry = doc["retry"]
    hconns = gc.pin_free(hconns, doc["initial_units"], {int(k2): v for k2, v in retry["free_per_level"].items()})
    cs = {s.name: s for s in static.conn_fields}
    dconns = tuple({n: to_column(v, cs[n], DEV) for n, v in b.items()} for b in hconns)
    r2 = phase.retry(k, units, dconns, tail_start=0)
    got = [{n: column_to_numpy(v, cs[n]) for n, v in b.items()} for b in r2.conns]
    assert gc.grown_pairs(hconns, got) == gc.want_commits(retry["expect"])
    assert r2.overflow == retry["expect"]["conn_overflow"]
    assert out.grown + r2.grown == doc["step_growth"]["expect"]["grown"]


def _state_from_host(static, units, conns, **flags) -> NetworkState:
    us = {s.name: s for s in static.unit_fields}
    cs = {s.name: s for s in static.conn_fields}
    return NetworkState({k: to_column(v, us[k], DEV) for k, v in units.items()},
                        tuple({k: to_column(v, cs[k], DEV) for k, v in b.items()} for b in conns), None, **flags)


@pytest.mark.parametrize("seed", [0, 1])
def test_device_resort_matches_oracle(seed: int) -> None:
    import test_resort_oracle as tro

    rng = np.random.default_rng(20 + seed)
    n, n_in = 2000, 16
    src, dst = tro._random_dag(rng, n, 8000, n_in)
    static, units, conns = tro._build(n, src, dst, range(n_in))
    for c in conns:
        live = np.flatnonzero(~c["dead"].astype(bool))
        c["dead"][live[rng.random(live.size) < 0.2]] = True
    b0 = conns[0]
    free = np.flatnonzero(b0["dead"].astype(bool))[:20]
    deep = np.argsort(units["level"])[-20:]
    b0["from_id"][free], b0["to_id"][free], b0["dead"][free] = rng.integers(0, n_in, 20), deep, False
    ref = og.resort(static, units, conns)
    st = _state_from_host(static, units, conns, needs_resort=True)
    new_static, new_state = device_resort(static, st)
    assert new_static.level_capacities == ref[0].level_capacities
    us = {s.name: s for s in static.unit_fields}
    cs = {s.name: s for s in static.conn_fields}
    assert np.array_equal(column_to_numpy(new_state.units["level"], us["level"]), ref[1]["level"])
    got = [{k: column_to_numpy(v, cs[k]) for k, v in b.items()} for b in new_state.conns]
    _same_arena(got, ref[2])
    assert not new_state.needs_resort


class AnyDirProposal(px.ProposeAddConn):
    """Proposals towards higher ids only (the id order stays topological, so
    no cycle), same level allowed: the commits raise needs_resort."""

    proposer = "per_unit"
    proposals_per_proposer = 3
    max_new_per_level = 25
    max_level_gap = 1
    direction = "same_or_deeper"

    def propose(self, u, i, j, g, rng):
        step = rng.uniform_int(48).astype(jnp.int32) + jnp.int32(1)
        return jnp.asarray(i, jnp.int32), jnp.asarray(i, jnp.int32) + step, rng.uniform()

    def init(self, u, src, dst, g):
        return px.ConnWrite.of((px.WEIGHT, jnp.float32(0.01)))


@pytest.mark.parametrize("pipeline", [False, True])
def test_driver_regrow_retry_and_resort_bit_exact(oracle, pipeline: bool) -> None:
    rng = np.random.default_rng(31 + pipeline)
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT)
    layers = [24, 120, 120, 8]
    base = np.concatenate([[0], np.cumsum(layers)])
    n = int(base[-1])
    src, dst = [], []
    for l in range(len(layers) - 1):
        a = np.arange(base[l], base[l + 1])
        b = np.arange(base[l + 1], base[l + 2])
        m = rng.random((a.size, b.size)) < 0.2
        ii, jj = np.nonzero(m)
        src.append(a[ii])
        dst.append(b[jj])
    src = np.concatenate(src).astype(np.int32)
    dst = np.concatenate(dst).astype(np.int32)
    w = (rng.standard_normal(src.size) * 0.2).astype(np.float32)

    class Net(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        add_conn = AnyDirProposal()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        extra_conn_fields = tuple(opt.state_fields)
        propagation = px.Propagation.PIPELINE if pipeline else px.Propagation.TOPOLOGICAL

    ins, outs = np.arange(layers[0]), np.arange(n - layers[-1], n)
    static, state = px.NetworkBuilder.from_edges(
        Net, n, src, dst, weights=w, input_ids=ins, output_ids=outs, globals_=None,
        capacity_headroom=0.02, device="cuda")
    o = nets.oracle_for(oracle, Net, static, state)
    o.tail_start = int(state.tail_start)
    if px.make_step(Net, static).backward_order == "slot":
        o.tile = None  # growth every step: the churn layout's slot-order backward
    od = oracle.OracleDriver(o)
    drv = Driver(Net, static, state)
    xs = rng.standard_normal((12, layers[0])).astype(np.float32)
    teacher = rng.standard_normal((layers[-1], layers[0])).astype(np.float32) * np.float32(0.2)
    for k in range(1, 11):
        x = xs[k - 1]
        t = np.tanh(teacher @ x).astype(np.float32)
        print(f"driver step {k} pipeline={pipeline}", flush=True)
        res = drv.step(px.StepInputs(x, t))
        lo = od.step(x, t)
        st = drv.state
        assert drv.static.level_capacities == o.static.level_capacities, f"capacities at step {k}"
        assert (st.grown, st.overflow, st.needs_resort, st.tail_start) == (
            o.grown, o.overflow, o.needs_resort, o.tail_start), f"flags at step {k}"
        torch.cuda.synchronize()
        assert_same_state(drv.static, st, o, f"step {k}")
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at {k}"
    assert drv.regrows > 0
    if not pipeline:
        assert drv.resorts > 0
