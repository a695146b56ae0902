"""Fused forward + prune on the device (phases.py:2322-2469): bit-identical
to the two-pass step, and to the oracle, over churn steps.

Each net runs four ways from the same state: ``fuse_prune="off"`` (the
predicate pass at the prune slot), ``"triton"`` (the predicate evaluated
inside plx_forward_bucket's sweep, tombstones committed at the prune slot),
``"xla"`` (the predicate pass at the forward's slot) and ``"auto"``; the
"triton" run takes the predicate compiled into the forward kernel and is
repeated with the predicate interpreted there. Every unit column, every
logical connection column, the loss and the structural flags must agree bit
for bit at every step, and the fused run must match the oracle (whose prune
runs at its own slot). Cases, after the reference's tests/test_prune_fusion.py:
an edge-column hash predicate with training and gradient-scored regrowth; the
same under PIPELINE propagation with per-unit proposals; a magnitude prune
without update_conn; a predicate on a field the forward writes from an
unwritten column and the globals (forwarded, computed before the sweep).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import nets
import plastax_amd as px
from test_fusion_plan import MARK, MASK, HashPrune, MarkedPrune, MarkForward, WeightPrune
from test_gpu_parity import _equal, assert_same_state
from test_gpu_structural_step import GradGrow, Propose4, _sparse_mlp

pytestmark = pytest.mark.gpu


def _net(prune, *, forward=None, train=True, grow=None, pipeline=False):
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT)

    class Net(px.Network):
        forward_pass = forward or nets.TanhForward()
        loss = nets.MSELoss() if train else None
        backward_pass = nets.TanhBackward() if train else None
        update_conn = opt.update_conn() if train else None
        prune_conn = prune
        add_conn = grow
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD, MARK, MASK)
        extra_conn_fields = tuple(opt.state_fields) if train else ()
        propagation = px.Propagation.PIPELINE if pipeline else px.Propagation.TOPOLOGICAL

    return Net


def _build(net, pipeline: bool, seed: int):
    rng = np.random.default_rng(seed)
    if pipeline:
        n = 1024
        src = rng.integers(0, n, 6000).astype(np.int32)
        dst = rng.integers(0, n, 6000).astype(np.int32)
        keep = src != dst
        src, dst = src[keep], dst[keep]
        w = (rng.standard_normal(src.size) * 0.3).astype(np.float32)
        ins, outs = np.arange(32), np.arange(n - 16, n)
    else:
        n, src, dst, w, ins, outs = _sparse_mlp(rng, [48, 160, 160, 16], 0.15)
    g = {"step": np.int32(0), "tau": np.float32(0.0), "scale": np.float32(1.0)}
    static, state = px.NetworkBuilder.from_edges(
        net, n, src, dst, weights=w, input_ids=ins, output_ids=outs, globals_=g, capacity_headroom=0.5,
        device="cuda")
    mask = (rng.random(n) < 0.1).astype(np.float32)
    units = dict(state.units)
    units[MASK.name] = torch.from_numpy(mask).to("cuda")
    state.units = units
    return static, state, len(ins), len(outs)


def _clone(state):
    return px.NetworkState({k: v.clone() for k, v in state.units.items()},
                           tuple({k: v.clone() for k, v in b.items()} for b in state.conns), state.globals_,
                           state.needs_resort, state.step, state.grown, state.overflow, state.units_added,
                           state.unit_overflow, state.tail_start)


def _host(static, state):
    return nets.host_units(static, state), nets.host_conns(static, state)


@pytest.mark.parametrize(
    "case",
    ["hash+train+grow", "hash+pipeline+propose", "weight, no update", "marked (forwarded)"],
)
def test_fused_step_matches_two_pass_and_oracle(oracle, case: str, monkeypatch) -> None:
    pipeline = case == "hash+pipeline+propose"
    if case == "hash+train+grow":
        net = _net(HashPrune(), grow=GradGrow())
    elif pipeline:
        net = _net(HashPrune(), grow=Propose4(), pipeline=True)
    elif case == "weight, no update":
        net = _net(WeightPrune(), train=False)
    else:
        net = _net(MarkedPrune(), forward=MarkForward())
    static, state0, n_in, n_out = _build(net, pipeline, 21)
    runs = {}
    rng = np.random.default_rng(5)
    xs = rng.standard_normal((8, n_in)).astype(np.float32)
    ts = np.tanh(rng.standard_normal((8, n_out))).astype(np.float32)
    o = nets.oracle_for(oracle, net, static, state0)
    o.tail_start, o.needs_resort = int(state0.tail_start), bool(state0.needs_resort)
    from plastax_amd import step as step_mod

    for mode in ("off", "triton", "triton/interpreted", "xla", "auto"):
        state = _clone(state0)
        engine = mode.split("/")[0]
        monkeypatch.setattr(step_mod, "FUSED_PREDICATE", "interpreted" if mode.endswith("interpreted") else "compiled")
        step = px.make_step(net, static, fuse_prune=engine)
        if step.backward_order == "slot":
            o.tile = None
        trace = []
        for k in range(8):
            g = {"step": np.int32(k), "tau": np.float32(0.05 * (k % 2)), "scale": np.float32(1.0)}
            state.globals_ = g
            print(f"fusion {case} {mode} step {k}", flush=True)
            res = step(state, px.StepInputs(xs[k], ts[k] if net.loss is not None else None))
            state = res.state
            trace.append((float(res.loss), state.grown, state.overflow, state.tail_start))
            if mode == "triton":
                o.globals_ = g
                lo = o.step(xs[k], ts[k] if net.loss is not None else None)
                assert (state.grown, state.overflow, state.tail_start) == (o.grown, o.overflow, o.tail_start)
                torch.cuda.synchronize()
                assert_same_state(static, state, o, f"{case} step {k}")
                assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at {k}"
        plan = step.prune_fusion.plan
        if engine == "off":
            assert plan is not None and not plan.fused
        elif engine == "auto":
            assert plan is not None and plan.fused == (plan.engine == "hip"), plan
        else:
            assert plan.fused and plan.engine == ("hip" if engine == "triton" else "xla"), plan
        if plan.fused and plan.engine == "hip":
            # the predicate compiled into the forward kernel, or interpreted there
            assert (step._fused_handle is not None) == (mode != "triton/interpreted"), mode
        runs[mode] = (trace, _host(static, state))
    for mode in ("triton", "triton/interpreted", "xla", "auto"):
        assert runs[mode][0] == runs["off"][0], mode
        (ua, ca), (ub, cb) = runs[mode][1], runs["off"][1]
        for name in ua:
            assert np.array_equal(ua[name].view(np.uint8), ub[name].view(np.uint8)), (mode, name)
        for a, b in zip(ca, cb):
            for name in a:
                assert np.array_equal(np.asarray(a[name]).view(np.uint8), np.asarray(b[name]).view(np.uint8)), \
                    (mode, name)
    dead = np.concatenate([c["dead"] for c in runs["triton"][1][1]])
    dead0 = np.concatenate([np.asarray(c["dead"].cpu()) for c in state0.conns])
    assert int(dead.sum()) > int(dead0.sum()), "nothing was pruned"


def test_compiled_forward_refuses_a_mismatched_descriptor() -> None:
    """plx_forward_bucket_compiled checks the descriptor against what the
    kernel was compiled for (monoid, the id arrays its shape reads) and
    launches nothing when they differ."""
    import ctypes

    from plastax_amd import _lib, _site, grow

    udt = {"activation": np.dtype(np.float32), "level": np.dtype(np.int32)}
    cdt = {"from_id": np.dtype(np.int32), "to_id": np.dtype(np.int32), "weight": np.dtype(np.float32)}
    sp = _site.trace_predicate(HashPrune(), udt, cdt, {"step": np.int32(0)})
    prog = _lib.plx_site_prog()
    code = sp.flat_code().reshape(-1, 4)
    prog.ninstr, prog.nout = len(code), len(sp.out_kinds)
    for k, row in enumerate(code):
        for j in range(4):
            prog.code[4 * k + j] = int(row[j])
    dev = torch.device("cuda", 0)
    handle = grow.compiled_forward_prune_handle(sp, prog, 0, dev)
    assert handle is not None
    lib = _lib.load()
    d = _lib.plx_forward_desc()
    d.nrows, d.monoid = 1, 0
    d.prune_prog = 16  # (never dereferenced: every check below fails first)
    assert lib.plx_forward_bucket_compiled(ctypes.c_void_p(handle), ctypes.byref(d), None) != 0  # no id arrays
    assert "compiled shape" in lib.plx_last_error().decode()
    d.monoid = 2
    assert lib.plx_forward_bucket_compiled(ctypes.c_void_p(handle), ctypes.byref(d), None) != 0
    assert "monoid" in lib.plx_last_error().decode()
