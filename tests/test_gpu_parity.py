"""Device parity: the HIP path against the CPU oracle, through the C ABI.

Integer and bit-level quantities (Philox words) and every float32 value of a
trajectory must match bit for bit: the kernels fold in the oracle's order and
evaluate the same float32 operation sequence (the library is built without
contraction, and exp/log/tanh follow the same published algorithm on both
sides). Where an exact match would be too strong a claim -- none here -- the
tolerance is written in the test.
"""

from __future__ import annotations

import os

import ctypes

import numpy as np
import pytest
import torch

import nets
import plastax_amd as px
from plastax_amd import _lib, synth
from plastax_amd.state import column_to_numpy

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _equal(a: np.ndarray, b: np.ndarray) -> bool:
    """Bitwise equality of float arrays (NaN == NaN, -0.0 != +0.0)."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    if a.dtype == np.float32:
        return a.shape == b.shape and bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))
    return bool(np.array_equal(a, b))


def _first_diff(a: np.ndarray, b: np.ndarray) -> str:
    bad = np.flatnonzero(a.view(np.uint32) != b.view(np.uint32)) if a.dtype == np.float32 else np.flatnonzero(a != b)
    if bad.size == 0:
        return "shapes differ"
    i = bad[0]
    return f"{bad.size} differ; first at {i}: device {a[i]!r} oracle {b[i]!r}"


def assert_same_state(static, state, o, what: str) -> None:
    for s in static.unit_fields:
        got = column_to_numpy(state.units[s.name], s)
        assert _equal(got, o.units[s.name]), f"{what}: unit {s.name}: {_first_diff(got, o.units[s.name])}"
    specs = {s.name: s for s in static.conn_fields}
    for b, bucket in enumerate(state.conns):
        for name, spec in specs.items():
            got = column_to_numpy(bucket[name], spec)
            ref = o.conns[b][name]
            assert _equal(got, ref), f"{what}: bucket {b} {name}: {_first_diff(got, ref)}"


# ---------------------------------------------------------------------------
# Elementary functions and Philox.
# ---------------------------------------------------------------------------


def _device_math(op: int, x: np.ndarray, y: np.ndarray | None = None) -> np.ndarray:
    xt = torch.from_numpy(x).to(DEV)
    yt = torch.from_numpy(y).to(DEV) if y is not None else None
    out = torch.empty_like(xt)
    _lib.call("plx_eval_math", op, x.size, xt.data_ptr(), yt.data_ptr() if yt is not None else None,
              out.data_ptr(), None)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_device_math_is_bit_exact_with_the_oracle(oracle) -> None:
    lib = oracle.load()
    rng = np.random.default_rng(0)
    specials = np.asarray([0.0, -0.0, 1.0, -1.0, 0.625, -0.625, 88.7, -103.9, 1e-40, -1e-40,
                           np.inf, -np.inf, np.nan, 44.4, -44.4, 1e-30, 8192.5, -3e7, 16777215.0,
                           np.pi, np.pi / 2], dtype=np.float32)
    xs = np.concatenate([
        rng.uniform(-90, 90, 20000), rng.uniform(-2, 2, 20000), rng.standard_normal(20000),
        np.exp(rng.uniform(-80, 80, 20000)), specials,
    ]).astype(np.float32)
    for op, fn in ((0, lib.ox_expf), (2, lib.ox_tanhf), (3, lib.ox_sigmoidf), (6, lib.ox_cosf), (7, lib.ox_sinf),
                   (8, lib.ox_log1pf), (9, lib.ox_expm1f)):
        dev = _device_math(op, xs)
        ref = np.asarray([fn(float(v)) for v in xs], dtype=np.float32)
        assert _equal(dev, ref), f"op {op}: {_first_diff(dev, ref)}"
    pos = np.abs(xs)
    dev = _device_math(1, pos)
    ref = np.asarray([lib.ox_logf(float(v)) for v in pos], dtype=np.float32)
    assert _equal(dev, ref), f"log: {_first_diff(dev, ref)}"
    dev = _device_math(4, pos)
    assert _equal(dev, np.sqrt(pos)), "sqrt must be correctly rounded"
    b = np.full(5000, np.float32(0.999), np.float32)
    b[::2] = np.float32(0.9)
    t = rng.integers(0, 200000, 5000).astype(np.float32)
    t[:3] = [0.5, 1.25, 70000.0]
    dev = _device_math(5, b, t)
    ref = np.asarray([lib.ox_pow_step(float(bb), float(tt)) for bb, tt in zip(b, t)], np.float32)
    assert _equal(dev[3:], ref[3:]), f"pow: {_first_diff(dev[3:], ref[3:])}"
    np.testing.assert_allclose(dev[:3], ref[:3], rtol=2e-7)  # non-integer t: device powf


def test_device_philox_is_bit_exact_with_the_oracle(oracle) -> None:
    rng = np.random.default_rng(1)
    seeds = rng.integers(0, 2**63, 4096, dtype=np.int64).astype(np.uint64)
    ctrs = rng.integers(0, 2**63, 4096, dtype=np.int64).astype(np.uint64)
    seeds[:2] = [0, 0xFFFFFFFFFFFFFFFF]
    ctrs[:2] = [0, 0xFFFFFFFFFFFFFFFF]
    s = torch.from_numpy(seeds.view(np.int64)).to(DEV)
    c = torch.from_numpy(ctrs.view(np.int64)).to(DEV)
    out = torch.empty(4096, dtype=torch.int32, device=DEV)
    _lib.call("plx_philox32", 4096, s.data_ptr(), c.data_ptr(), out.data_ptr(), None)
    dev = out.cpu().numpy().view(np.uint32)
    ref = np.asarray([oracle.load().ox_philox32(int(a), int(b)) for a, b in zip(seeds, ctrs)], np.uint32)
    assert np.array_equal(dev, ref)
    assert dev[0] == 0x6627E8D5 and dev[1] == 0x408F276D  # Random123 KATs
    assert np.array_equal(px.rng.philox32(seeds, ctrs), ref)


# ---------------------------------------------------------------------------
# Goldens through the device step.
# ---------------------------------------------------------------------------


def test_passes_relu_topological_golden_on_device() -> None:
    doc = nets.load_golden("passes_relu_topological.json")
    static, state = nets.build_golden(nets.ReluMlpNet, doc, device="cuda")
    step = px.make_step(nets.ReluMlpNet, static)
    for i, s in enumerate(doc["steps"]):
        res = step(state, px.StepInputs(np.float32(s["inputs"]), np.float32(s["targets"])))
        state = res.state
        assert state.units["activation"].cpu().tolist() == s["expect"]["activations"], i
        assert state.units["grad_pre_act"].cpu().tolist() == s["expect"]["grad_pre_act"], i
        assert float(res.loss) == s["expect"]["loss"], i


def test_passes_relu_pipeline_golden_on_device() -> None:
    doc = nets.load_golden("passes_relu_pipeline.json")
    static, state = nets.build_golden(nets.ReluPipelineNet, doc, device="cuda")
    step = px.make_step(nets.ReluPipelineNet, static)
    for i, s in enumerate(doc["steps"]):
        state = step(state, px.StepInputs(np.float32(s["inputs"]))).state
        assert state.units["activation"].cpu().tolist() == s["expect"]["activations"], i


@pytest.mark.parametrize("name", [
    "loss_softmax_ce_large_logits", "loss_softmax_ce_negative_logits",
    "loss_softmax_ce_one_hot", "loss_softmax_ce_soft_targets", "loss_softmax_ce_tied_max",
])
def test_softmax_ce_golden_on_device(name: str) -> None:
    doc = nets.load_golden(f"{name}.json")
    static, state = nets.build_golden(nets.SoftmaxNet, doc, device="cuda")
    out = list(static.output_ids)
    step = px.make_step(nets.SoftmaxNet, static)
    for i, s in enumerate(doc["steps"]):
        res = step(state, px.StepInputs(np.float32(s["inputs"]), np.float32(s["targets"])))
        state = res.state
        assert state.units["activation"].cpu().numpy()[out].tolist() == s["expect"]["activations"]
        assert state.units["loss_grad"].cpu().numpy()[out].tolist() == s["expect"]["seed"], i
        assert float(res.loss) == s["expect"]["loss"], i


# ---------------------------------------------------------------------------
# Trajectories: device vs oracle, bit for bit.
# ---------------------------------------------------------------------------


def _run_both(net, static, state, oracle, inputs_fn, steps, check_at, tile=None, nsuper=None,
              parallel=False):
    kw = {} if tile is None else {"tile": tile}
    if nsuper is not None:
        kw["nsuper"] = nsuper
    o = nets.oracle_for(oracle, net, static, state, parallel=parallel, **kw)
    if parallel:
        o.lib.ox_set_threads(min(16, len(os.sched_getaffinity(0))))
    step = px.make_step(net, static)
    if tile is not None:
        step.tile = tile
    if nsuper is not None:
        step.nsuper = nsuper
    for k in range(1, steps + 1):
        x, t = inputs_fn(k)
        res = step(state, px.StepInputs(x, t))
        state = res.state
        lo = o.step(x, t)
        if k in check_at:
            torch.cuda.synchronize()
            assert_same_state(static, state, o, f"step {k}")
            assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at {k}"
            print(f"step {k}: every column bit-exact", flush=True)
    if parallel:
        o.lib.ox_set_threads(1)
    return state, o


def test_c1_pipeline_sgd_1000_steps_bit_exact(oracle) -> None:
    """C1: recurrent pipeline, tanh, SGD lr 1e-2, 1,000 steps."""
    e = synth.c1_pipeline(0)
    net = nets.make_trained_net("C1", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.sgd(1e-2, nets.GRAD_PRE_ACT), px.Propagation.PIPELINE)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cuda")
    a = synth.c1_target(0)
    rng = np.random.default_rng(7)
    xs = rng.standard_normal((1000, 32)).astype(np.float32)

    def inputs(k):
        x = xs[k - 1]
        return x, (a @ x).astype(np.float32)

    _run_both(net, static, state, oracle, inputs, 1000, {1, 10, 100, 1000})


@pytest.mark.parametrize("opt_name", ["adam", "adamw", "sgd", "momentum", "rmsprop"])
def test_topological_zipf_net_bit_exact(oracle, opt_name: str) -> None:
    """A C2-shaped net at 1/64 width (8 layers x 2,048 units, ~1M edges)."""
    opt = {
        "adam": px.optim.adam(1e-3, nets.GRAD_PRE_ACT),
        "adamw": px.optim.adamw(1e-3, nets.GRAD_PRE_ACT, weight_decay=1e-2),
        "sgd": px.optim.sgd(1e-2, nets.GRAD_PRE_ACT),
        "momentum": px.optim.momentum(1e-2, 0.9, nets.GRAD_PRE_ACT),
        "rmsprop": px.optim.rmsprop(1e-3, nets.GRAD_PRE_ACT),
    }[opt_name]
    e = synth.c2_topological(seed=3, scale=64)
    net = nets.make_trained_net(f"Z_{opt_name}", nets.TanhForward(), nets.TanhBackward(), opt,
                                px.Propagation.TOPOLOGICAL)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, capacity_align=256, device="cuda")
    width = e.input_ids.size
    sign, perm = synth.c2_target(3, width)
    rng = np.random.default_rng(11)

    def inputs(k):
        x = rng.standard_normal(width).astype(np.float32)
        return x, (sign * x[perm]).astype(np.float32)

    _run_both(net, static, state, oracle, inputs, 12, {1, 12})


def test_c2_generator_adam_1000_steps_bit_exact(oracle) -> None:
    """C2's generator at 1/64 width (8 layers x 2,048 tanh units, ~1M Zipf
    edges), MSE, Adam(1e-3), 1,000 streaming steps: every unit and
    connection column and the loss equal the oracle's at steps 1, 10, 100
    and 1,000."""
    e = synth.c2_topological(seed=5, scale=64)
    net = nets.make_trained_net("Z1000", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.adam(1e-3, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, capacity_align=256, device="cuda")
    width = e.input_ids.size
    sign, perm = synth.c2_target(5, width)
    rng = np.random.default_rng(13)
    xs = rng.standard_normal((1000, width)).astype(np.float32)

    def inputs(k):
        x = xs[k - 1]
        return x, (sign * x[perm]).astype(np.float32)

    _run_both(net, static, state, oracle, inputs, 1000, {1, 10, 100, 1000}, parallel=True)


@pytest.mark.parametrize("tile,nsuper", [(64, 512), (1024, 512), (64, 5), (256, 37)])
def test_many_tiles_and_hot_sources_bit_exact(oracle, tile: int, nsuper: int) -> None:
    """Small tiles: many tiles per superblock, the Zipf head lands in the
    workgroups' hot running sums and the tail in the cold runs."""
    e = synth.c2_topological(seed=8, scale=128)
    net = nets.make_trained_net(f"T{tile}", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.adam(1e-3, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cuda")
    width = e.input_ids.size
    rng = np.random.default_rng(12)

    def inputs(k):
        x = rng.standard_normal(width).astype(np.float32)
        return x, np.tanh(x[::-1]).astype(np.float32)

    _run_both(net, static, state, oracle, inputs, 6, {1, 6}, tile=tile, nsuper=nsuper)


@pytest.mark.parametrize("tile,nsuper", [(128, 512), (128, 3)])
def test_hub_groups_over_many_ranks_bit_exact(oracle, tile: int, nsuper: int) -> None:
    """Short rows under hub sources: a hub's (tile, source) group spans 15 or
    more ranks, so its end comes from the rank tags' start bits."""
    e = nets.hub_edges(5)
    net = nets.make_trained_net(f"H{nsuper}", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.adam(1e-3, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cuda")
    width, n_out = e.input_ids.size, e.output_ids.size
    rng = np.random.default_rng(14)

    def inputs(k):
        x = rng.standard_normal(width).astype(np.float32)
        return x, np.tanh(x[:n_out]).astype(np.float32)

    _run_both(net, static, state, oracle, inputs, 6, {1, 6}, tile=tile, nsuper=nsuper)


def test_strided_inputs_and_targets(oracle) -> None:
    """Inputs and targets given as strided views (rows of column-major
    arrays, as numpy's fancy indexing returns) step exactly like dense
    copies: the kernels read dense arrays, so the step copies such views."""
    e = synth.c2_topological(seed=12, scale=256)
    net = nets.make_trained_net("SV", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.adam(1e-3, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    width = e.input_ids.size
    rng = np.random.default_rng(15)
    xs = np.asfortranarray(rng.standard_normal((3, width)).astype(np.float32))
    ts = np.asfortranarray(np.tanh(xs[:, ::-1]).astype(np.float32))
    xs_d, ts_d = torch.from_numpy(xs).to("cuda"), torch.from_numpy(ts).to("cuda")
    assert not xs_d[1].is_contiguous() and not ts_d[1].is_contiguous()
    losses = []
    for strided in (True, False):
        static, state = px.NetworkBuilder.from_edges(
            net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
            output_ids=e.output_ids, globals_=None, device="cuda")
        step = px.make_step(net, static)
        got = []
        for k in range(3):
            x, t = (xs_d[k], ts_d[k]) if strided else (xs_d[k].contiguous(), ts_d[k].contiguous())
            res = step(state, px.StepInputs(x, t))
            state = res.state
            got.append(float(res.loss))
        losses.append(got)
    assert losses[0] == losses[1]
    o = nets.oracle_for(oracle, net, static, px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cpu")[1])
    want = [float(o.step(np.ascontiguousarray(xs[k]), np.ascontiguousarray(ts[k]))) for k in range(3)]
    assert losses[0] == want


def test_dead_slots_and_headroom_bit_exact(oracle) -> None:
    """Tombstoned slots inside rows and a capacity tail are skipped by every
    pass and never written."""
    e = synth.c2_topological(seed=10, scale=256)
    net = nets.make_trained_net("DS", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.momentum(1e-2, 0.9, nets.GRAD_PRE_ACT),
                                px.Propagation.TOPOLOGICAL)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cuda", capacity_headroom=0.3,
        capacity_align=12)
    for bucket in state.conns:
        live = torch.nonzero(bucket["dead"] == 0).flatten()
        bucket["dead"][live[::5]] = 1
    width = e.input_ids.size
    rng = np.random.default_rng(13)

    def inputs(k):
        x = rng.standard_normal(width).astype(np.float32)
        return x, x[::-1].copy()

    _run_both(net, static, state, oracle, inputs, 4, {1, 4}, tile=512)


@pytest.mark.parametrize("dead", [False, True])
def test_forward_blocks_beyond_the_persistent_grid(oracle, dead: bool) -> None:
    """A level of more rows than the forward's persistent grid covers in one
    pass (cu_count x 2 workgroups x 256 rows): workgroups take two row blocks
    each, so the next block's prefetch and row set-up run. With `dead`,
    tombstones inside the rows make the forward read the DEAD column."""
    cu = torch.cuda.get_device_properties(0).multi_processor_count
    wide = cu * 2 * 256 * 3 // 2 + 77
    widths = (1024, wide, 24)
    rng = np.random.default_rng(21)
    base = np.cumsum([0, *widths])
    src = [base[0] + rng.integers(0, widths[0], (wide, 3)).ravel()]
    dst = [np.repeat(np.arange(base[1], base[2]), 3)]
    src.append(base[1] + rng.integers(0, wide, (widths[2], 400)).ravel())
    dst.append(np.repeat(np.arange(base[2], base[3]), 400))
    src = np.concatenate(src).astype(np.int32)
    dst = np.concatenate(dst).astype(np.int32)
    fan = np.bincount(dst, minlength=int(base[-1]))
    w = (rng.standard_normal(src.size) / np.sqrt(fan[dst])).astype(np.float32)
    net = nets.make_trained_net(f"Wide{int(dead)}", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.adam(1e-3, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state = px.NetworkBuilder.from_edges(
        net, int(base[-1]), src, dst, weights=w, input_ids=np.arange(widths[0]),
        output_ids=np.arange(base[2], base[3]), globals_=None, device="cuda")
    if dead:
        for bucket in state.conns:
            live = torch.nonzero(bucket["dead"] == 0).flatten()
            bucket["dead"][live[::7]] = 1
    rng_x = np.random.default_rng(22)

    def inputs(k):
        x = rng_x.standard_normal(widths[0]).astype(np.float32)
        return x, np.tanh(x[: widths[2]]).astype(np.float32)

    print(f"wide forward: {wide} rows in bucket 0, {src.size} edges, dead={dead}", flush=True)
    _run_both(net, static, state, oracle, inputs, 3, {1, 3})


@pytest.mark.parametrize("fwd,bwd", [
    (nets.SigmoidForward(), nets.SigmoidBackward()),
    (nets.ReluForward(), nets.ReluBackward()),
    (nets.MaxForward(), nets.TanhBackward()),
])
def test_other_policies_bit_exact(oracle, fwd, bwd) -> None:
    e = synth.c2_topological(seed=5, scale=256)
    net = nets.make_trained_net("P_" + type(fwd).__name__, fwd, bwd,
                                px.optim.adam(1e-3, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cuda")
    width = e.input_ids.size
    rng = np.random.default_rng(2)

    def inputs(k):
        x = rng.standard_normal(width).astype(np.float32)
        return x, np.tanh(x[::-1]).astype(np.float32)

    _run_both(net, static, state, oracle, inputs, 5, {1, 5})


def test_device_step_is_deterministic() -> None:
    """Two runs from the same state give the same bits (no float atomics)."""
    e = synth.c2_topological(seed=9, scale=32)
    net = nets.make_trained_net("Det", nets.TanhForward(), nets.TanhBackward(),
                                px.optim.adam(1e-3, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    outs = []
    for _ in range(2):
        static, state = px.NetworkBuilder.from_edges(
            net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
            output_ids=e.output_ids, globals_=None, device="cuda")
        step = px.make_step(net, static)
        rng = np.random.default_rng(4)
        width = e.input_ids.size
        for _ in range(3):
            x = rng.standard_normal(width).astype(np.float32)
            state = step(state, px.StepInputs(x, x[::-1].copy())).state
        outs.append((state.units["activation"].cpu().numpy(),
                     state.conns[3]["weight"].cpu().numpy()))
    assert _equal(outs[0][0], outs[1][0]) and _equal(outs[0][1], outs[1][1])
