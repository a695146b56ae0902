"""The tiled arena built on the device (plastax_amd/_layout_dev.py) equals
the host build (plastax_amd/_layout.py) table for table.

Every field of the two arenas is compared exactly: the unit order, the slab
columns and slots, the forward rows and ranges, the one-byte destinations,
and per bucket the tiles, superblocks, sorted ranks, group descriptors, hot
range, tile info, cold slots and superblock ids, finalize rows and parts.
Nets: a C2-shaped layered net (Zipf sources, 1/64 width) with a small tile
and many superblocks; a sparse MLP with skip connections (rows carried
across buckets) and dead slots; a PIPELINE reservoir; a net with unit
capacity and pruned units; and a layout after growth and pruning on the
device.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import batched_cases as bc
import nets
import plastax_amd as px
from plastax_amd import synth
from plastax_amd._layout import Arena, BackwardTiles
from plastax_amd._layout_dev import DeviceArena

pytestmark = pytest.mark.gpu


def _eq(a, b, what):
    if isinstance(a, torch.Tensor):
        a, b = a.cpu().numpy(), b.cpu().numpy()
    if isinstance(a, np.ndarray):
        assert a.shape == b.shape and np.array_equal(a, b), what
    else:
        assert a == b, what


def _compare(static, state, *, tile=4096, nsuper=512):
    dev = state.device
    stream = int(torch.cuda.current_stream(dev).cuda_stream)
    host = Arena(static, state.units, state._conns, dev, tile=tile, nsuper=nsuper)
    devc = DeviceArena(static, state.units, state._conns, dev, stream, tile=tile, nsuper=nsuper)
    torch.cuda.synchronize()
    for name in ("uperm", "uinv", "lvl_start", "caps", "bases", "ends", "lives", "n_positions", "fwd_carry",
                 "bwd_carry"):
        _eq(getattr(host, name), getattr(devc, name), name)
    for name in ("input_ids", "output_ids", "is_input", "slot"):
        _eq(getattr(host, name), getattr(devc, name), name)
    for name in host.cols:
        _eq(host.cols[name], devc.cols[name], f"column {name}")
    for b in range(host.num_buckets):
        fh, fd = host.fwd[b], devc.fwd[b]
        _eq(fh.nrows, fd.nrows, f"fwd {b} nrows")
        _eq(fh.rows, fd.rows, f"fwd {b} rows")
        _eq(fh.ptr, fd.ptr, f"fwd {b} ptr")
        for name in ("dst8", "blk_dst0"):
            a, c = getattr(host, name)[b], getattr(devc, name)[b]
            assert (a is None) == (c is None), f"{name} {b}"
            if a is not None:
                _eq(a, c, f"{name} {b}")
        bh, bd = host.bwd[b], devc.bwd[b]
        for field in BackwardTiles.__dataclass_fields__:
            a, c = getattr(bh, field), getattr(bd, field)
            if field in ("hot_sb", "cold_partial"):  # outputs of the backward, sized only
                assert (a is None) == (c is None) and (a is None or a.shape == c.shape), f"bwd {b} {field}"
                continue
            assert (a is None) == (c is None), f"bwd {b} {field}"
            if a is not None:
                _eq(a, c, f"bwd {b} {field}")
    for field in ("nrows", "rows", "nparts", "part_rows"):
        _eq(getattr(host.top, field), getattr(devc.top, field), f"top {field}")
    return host


def test_c2_shaped_layout_equals_host_build() -> None:
    e = synth.c2_topological(seed=3, scale=64)
    opt = px.optim.adam(1e-3, nets.GRAD_PRE_ACT)

    class C2(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        extra_conn_fields = tuple(opt.state_fields)

    static, state = px.NetworkBuilder.from_edges(
        C2, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids, output_ids=e.output_ids,
        globals_=None, device="cuda")
    print("layout: c2 1/64", flush=True)
    _compare(static, state, tile=512, nsuper=64)
    _compare(static, state)


def test_skip_connections_and_dead_slots() -> None:
    opt = px.optim.sgd(0.05, nets.GRAD_PRE_ACT)
    net = bc.tanh_mse_net(opt)
    static, state = bc.build(net, [40, 96, 80, 12], 0.3, skip=0.1, seed=31, device="cuda", headroom=0.5)
    conns = [dict(c) for c in state.conns]
    rng = np.random.default_rng(2)
    for c in conns:  # tombstone a fifth of the slots
        kill = torch.from_numpy(rng.random(c["dead"].numel()) < 0.2).to("cuda")
        c["dead"] = (c["dead"].bool() | kill).to(c["dead"].dtype)
    state.conns = tuple(conns)
    print("layout: skip + dead", flush=True)
    _compare(static, state, tile=256, nsuper=16)


def test_pipeline_reservoir() -> None:
    rng = np.random.default_rng(7)
    n = 900
    src = rng.integers(0, n, 7000).astype(np.int32)
    dst = rng.integers(0, n, 7000).astype(np.int32)
    keep = src != dst
    src, dst = src[keep], dst[keep]

    class Res(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = nets.MSELoss()
        update_conn = px.optim.sgd(1e-2, nets.GRAD_PRE_ACT).update_conn()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        propagation = px.Propagation.PIPELINE

    static, state = px.NetworkBuilder.from_edges(
        Res, n, src, dst, weights=(rng.standard_normal(src.size) * 0.2).astype(np.float32),
        input_ids=np.arange(16), output_ids=np.arange(n - 8, n), globals_=None, capacity_headroom=0.25,
        device="cuda")
    print("layout: pipeline", flush=True)
    _compare(static, state, tile=1024, nsuper=8)


def test_layout_after_device_growth_and_prune(oracle) -> None:
    """The tiled layout rebuilt after structural steps: the device build
    runs in the step (the default), and its arena equals the host build of
    the same logical state."""
    from test_gpu_structural_step import _run, _sparse_mlp, GradGrow, TauPrune

    rng = np.random.default_rng(4)
    n, src, dst, w, ins, outs = _sparse_mlp(rng, [64, 160, 160, 10], 0.12)
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT)

    class DST(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        prune_conn = TauPrune()
        add_conn = GradGrow()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        extra_conn_fields = tuple(opt.state_fields)

    static, state = px.NetworkBuilder.from_edges(
        DST, n, src, dst, weights=w, input_ids=ins, output_ids=outs, globals_={"tau": np.float32(0.0)},
        capacity_headroom=0.25, device="cuda")
    teacher = rng.standard_normal((10, 64)).astype(np.float32) * np.float32(0.1)
    xs = rng.random((12, 64)).astype(np.float32)
    state, o, grown = _run(DST, static, state, oracle, lambda k: (xs[k - 1], np.tanh(teacher @ xs[k - 1])),
                           lambda k: {"tau": np.float32(0.02 if k % 5 == 1 else 0.0)}, 11, {6, 11})
    assert grown > 0
    state.conns  # write the arena back to the logical buckets
    print("layout: after growth", flush=True)
    _compare(static, state)


def test_sources_above_2_to_the_20() -> None:
    """Physical source ids past 2^20 (2^20 + 64 input units, each feeding one
    of 96 hidden units, which feed 8 outputs): the tile build's sort keys
    hold (source << 12 | position) in 64 bits, so bucket 1's sources, whose
    physical ids all lie above 2^20, keep their ids, and the arena equals
    the host build."""
    n_in, n_hid, n_out = (1 << 20) + 64, 96, 8
    rng = np.random.default_rng(5)
    src0 = np.arange(n_in, dtype=np.int32)
    dst0 = (n_in + rng.integers(0, n_hid, n_in)).astype(np.int32)
    src1 = np.repeat(np.arange(n_in, n_in + n_hid, dtype=np.int32), 4)
    dst1 = (n_in + n_hid + rng.integers(0, n_out, src1.size)).astype(np.int32)
    src = np.concatenate([src0, src1])
    dst = np.concatenate([dst0, dst1])
    w = (rng.standard_normal(src.size) * 0.1).astype(np.float32)
    opt = px.optim.adam(1e-3, nets.GRAD_PRE_ACT)
    net = nets.make_trained_net("Wide20", nets.TanhForward(), nets.TanhBackward(), opt,
                                px.Propagation.TOPOLOGICAL)
    static, state = px.NetworkBuilder.from_edges(
        net, n_in + n_hid + n_out, src, dst, weights=w, input_ids=np.arange(n_in),
        output_ids=np.arange(n_in + n_hid, n_in + n_hid + n_out), globals_=None, device="cuda")
    print("layout: sources above 2^20", flush=True)
    host = _compare(static, state, tile=128, nsuper=8)
    assert int(host.lvl_start[1]) >= 1 << 20
