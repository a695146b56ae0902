"""BASELINE configurations at their full shapes on the device, every unit and
connection column compared with the oracle bit for bit (the workloads are
bench.py's: the same generators, policies and inputs).

- C2: 8 x 131,072 tanh units, 2^26 Zipf edges, MSE, Adam; three streaming
  steps against the oracle's parallel form (the same folds as its
  sequential form; OpenMP on the host's cores).
- C3: the 784-4096-4096-10 sparse MLP at 10 % keep, softmax cross-entropy,
  Adam, two batched steps at B = 256 against the batched oracle.
- C5: the 65,536-unit reservoir (262,144 unit slots, 16M edge slots) with
  its whole recipe -- out-degree count, PruneUnit, AddUnit (the first step
  spawns 16 units), per-unit proposals P = 4 -- two steps.
"""

from __future__ import annotations

import os
import time

import numpy as np
import pytest
import torch

import plastax_amd as px
from plastax_amd import synth
from plastax_amd.state import column_to_numpy
from test_gpu_parity import _equal, _first_diff

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _say(msg: str, t0: float) -> None:
    print(f"[{time.perf_counter() - t0:6.1f} s] {msg}", flush=True)


def _host(static, state):
    us = {s.name: s for s in static.unit_fields}
    cs = {s.name: s for s in static.conn_fields}
    units = {n: np.ascontiguousarray(column_to_numpy(state.units[n], us[n])) for n in us}
    conns = [{n: np.ascontiguousarray(column_to_numpy(b[n], cs[n])) for n in cs} for b in state.conns]
    return units, conns


def _to_device(state, globals_):
    g = px.NetworkState({k: v.to(DEV) for k, v in state.units.items()},
                        tuple({k: v.to(DEV) for k, v in b.items()} for b in state.conns), globals_)
    g.tail_start = state.tail_start
    return g


def _compare(static, state, o, what: str) -> None:
    units, conns = _host(static, state)
    for n, got in units.items():
        assert _equal(got, o.units[n]), f"{what}: unit {n}: {_first_diff(got, o.units[n])}"
    for b, cols in enumerate(conns):
        for n, got in cols.items():
            assert _equal(got, o.conns[b][n]), f"{what}: bucket {b} {n}: {_first_diff(got, o.conns[b][n])}"


def test_c2_full_size_three_steps(oracle) -> None:
    from bench import build_c2
    from plastax_amd._plan import compile_plan

    t0 = time.perf_counter()
    net, e = build_c2(px, 0, 1)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, capacity_align=256, device="cpu")
    _say(f"C2 logical arena: {e.src.size} edges", t0)
    units, conns = _host(static, state)
    o = oracle.OracleNet(static, units, conns, compile_plan(net, static), None, parallel=True)
    o.lib.ox_set_threads(min(16, len(os.sched_getaffinity(0))))
    gstate = _to_device(state, None)
    del state
    step = px.make_step(net, static)
    width = e.input_ids.size
    sign, perm = synth.c2_target(0, width)
    rng = np.random.default_rng(2)
    xs = rng.standard_normal((3, width)).astype(np.float32)
    ts = np.ascontiguousarray((sign[None, :] * xs[:, perm]).astype(np.float32))
    for k in range(3):
        res = step(gstate, px.StepInputs(xs[k], ts[k]))
        gstate = res.state
        lo = o.step(xs[k], ts[k])
        torch.cuda.synchronize()
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at step {k + 1}"
        _say(f"C2 step {k + 1}: loss {lo} equal", t0)
    o.lib.ox_set_threads(1)
    _compare(static, gstate, o, "C2 step 3")
    _say("C2: every unit and connection column bit-exact after 3 steps", t0)


def test_c3_full_shape_two_batched_steps(oracle) -> None:
    from bench import build_c3
    from oracle import batched as ob
    from plastax_amd._plan import compile_plan

    t0 = time.perf_counter()
    B = 256
    net = build_c3(px)
    e = synth.c3_mlp(0)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cpu")
    units, conns = _host(static, state)
    o = oracle.OracleNet(static, units, conns, compile_plan(net, static), None)
    o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
    orc = ob.OracleBatch(o, B)
    gstate = _to_device(state, None)
    step = px.make_step(net, static, batch_size=B)
    xs, ys = synth.c3_batches(0, 2, B)
    _say(f"C3: {e.src.size} edges, B = {B}", t0)
    for k in range(2):
        res = step(gstate, px.StepInputs(xs[k], ys[k]))
        gstate = res.state
        lo = orc.step(xs[k], ys[k])
        torch.cuda.synchronize()
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at step {k + 1}"
        _compare(static, gstate, o, f"C3 step {k + 1}")
        _say(f"C3 step {k + 1}: every column bit-exact", t0)


def test_c5_full_size_two_steps_with_a_spawn(oracle) -> None:
    from bench import build_c5_recipe
    from plastax_amd._plan import compile_plan

    t0 = time.perf_counter()
    e = synth.c5_reservoir(0)
    net = build_c5_recipe(px, e.num_units, 262144, 1024, 16)

    def g_of(k):
        return {"spawn": np.float32(1.0 if k % 100 == 0 else 0.0)}

    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=g_of(0), capacity_headroom=3.0, device="cpu")
    units, conns = _host(static, state)
    o = oracle.OracleNet(static, units, conns, compile_plan(net, static), g_of(0), tile=None)
    o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
    gstate = _to_device(state, g_of(0))
    step = px.make_step(net, static)
    rng = np.random.default_rng(3)
    xs = rng.standard_normal((2, e.input_ids.size)).astype(np.float32)
    _say(f"C5: {e.src.size} live edges of {static.level_capacities[0]} slots", t0)
    added = []
    for k in range(2):
        gstate.globals_ = g_of(k)
        o.globals_ = g_of(k)
        gstate = step(gstate, px.StepInputs(xs[k])).state
        o.step(xs[k])
        got = (int(gstate.units_added), bool(gstate.unit_overflow), int(gstate.grown), bool(gstate.overflow),
               int(gstate.tail_start))
        want = (o.units_added, o.unit_overflow, o.grown, o.overflow, o.tail_start)
        assert got == want, f"flags at step {k + 1}: device {got} oracle {want}"
        added.append(got[0])
        torch.cuda.synchronize()
        _compare(static, gstate, o, f"C5 step {k + 1}")
        _say(f"C5 step {k + 1}: flags {got}, every column bit-exact", t0)
    assert added == [16, 0]  # step 1 spawned the 16-unit band
