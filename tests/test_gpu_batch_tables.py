"""The batched step's per-bucket tables built on the device
(plastax_amd/_batch_dev.py) against their host builds, entry for entry:
the backward's source rows and slot-ordered out-edge lists
(batched.batch_sources_host) and the batched update's tiles
(_layout.batch_tiles). Cases: a sparse MLP with skip edges, tiles dense
enough to be cut, tombstones inside the rows, the C3 shape, and a bucket
emptied of live edges."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import batched_cases as bc
import nets
import plastax_amd as px
from plastax_amd import _layout, synth
from plastax_amd._batch_dev import batch_sources_dev, batch_tiles_dev
from plastax_amd.batched import batch_sources_host

pytestmark = pytest.mark.gpu


def _net():
    opt = px.optim.adam(1e-2, nets.GRAD_PRE_ACT)

    class Net(px.Network):
        forward_pass = nets.TanhForward()
        backward_pass = nets.TanhBackward()
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        extra_conn_fields = tuple(opt.state_fields)
        batch_reduction = px.MeanFloatFirstRest()

    return Net


def _compare(arena, what: str) -> None:
    for b in range(arena.num_buckets):
        h = batch_sources_host(arena, b)
        d = batch_sources_dev(arena, b)
        assert d.nrows == h.nrows, f"{what} bucket {b}: rows {d.nrows} vs {h.nrows}"
        for name in ("rows", "ptr", "pos", "dst"):
            got, want = getattr(d, name).cpu().numpy(), getattr(h, name).cpu().numpy()
            assert np.array_equal(got, want), f"{what} bucket {b}: batch_sources.{name} differs"
        base, live = arena.bases[b], arena.lives[b]
        src = arena.cols["from_id"][base : base + live].cpu().numpy()
        dst = arena.cols["to_id"][base : base + live].cpu().numpy()
        th = _layout.batch_tiles(src, dst)
        td = batch_tiles_dev(arena, b)
        for name in ("tile_off", "tile_base", "pos"):
            assert np.array_equal(td[name].cpu().numpy().astype(np.int64), th[name].astype(np.int64)), \
                f"{what} bucket {b}: batch_tiles.{name} differs"
        assert np.array_equal(td["loc"].cpu().numpy().view(np.uint16), th["loc"]), f"{what} bucket {b}: loc"
    print(f"{what}: {arena.num_buckets} buckets equal", flush=True)


@pytest.mark.parametrize("layers,keep,skip", [([24, 40, 33, 8], 0.3, 0.1), ([70, 300, 200, 12], 0.9, 0.0)])
def test_device_tables_equal_the_host_build(layers, keep, skip) -> None:
    net = _net()
    static, state = bc.build(net, layers, keep, skip=skip, seed=4, device="cuda")
    step = px.make_step(net, static, batch_size=8)
    _compare(step.arena(state), f"mlp {layers}")


def test_tombstones_and_an_empty_bucket() -> None:
    net = _net()
    static, state = bc.build(net, [30, 50, 40, 6], 0.4, skip=0.1, seed=5, device="cuda")
    rng = np.random.default_rng(6)
    for i, bucket in enumerate(state.conns):
        dead = bucket["dead"]
        if i == 1:
            dead.fill_(1)  # every edge of bucket 1 dead
        else:
            kill = torch.from_numpy(rng.random(dead.numel()) < 0.3).to(dead.device)
            dead[kill] = 1
    step = px.make_step(net, static, batch_size=4)
    _compare(step.arena(state), "tombstones")


def test_c3_shape() -> None:
    from bench import build_c3

    net = build_c3(px)
    e = synth.c3_mlp(0)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cuda")
    step = px.make_step(net, static, batch_size=256)
    _compare(step.arena(state), "C3")
