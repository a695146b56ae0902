"""Named monoids other than sum on the device, against the oracle bit for bit
(monoid.py:29-51, :84-122; the oracle's folds are pinned against numpy's
scatter ufuncs in test_monoid_oracle.py).

- forward (k_forward): max_, min_ and prod folds of w * x[src] per
  destination, on a Zipf net (multi-window rows, busiest-source tables) and
  on short rows under hub sources;
- backward (k_tile + k_finalize): max_, min_ and prod folds of w * g[dst]
  per source, with one tile per superblock and with small tiles (hot running
  sums, cold partials, groups over many ranks);
- tombstones inside rows and rows with no live term (the identity reaches
  the apply);
- PIPELINE, batched one-wave rows (k_forward_batch4 / k_backward_batch4) and
  a generic tuple pass (plx_gen_fold) with (min, prod, max) components.

The applies keep every value finite (a clamp of the identity where a row can
be empty), so the comparisons are plain uint32 equality.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import generic_cases as gc
import nets
import plastax_amd as px
import plastax_amd.numpy as jnp
from plastax_amd import synth
from test_gpu_parity import _equal, _run_both, assert_same_state

pytestmark = pytest.mark.gpu

MONOIDS = {"max": px.monoid.max_, "min": px.monoid.min_, "prod": px.monoid.prod}


def _forward(name: str):
    class Fwd(px.ForwardPass):
        combine = MONOIDS[name]

        def map(self, u, dst, src, c, cid, g):
            return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)))

    Fwd.__name__ = f"Fwd_{name}"
    return Fwd()


def _backward(name: str):
    """w * g[dst] folded by the monoid; the apply clamps an empty row's
    identity (max: -inf, min: +inf) to a finite value."""

    class Bwd(px.BackwardPass):
        combine = MONOIDS[name]

        def map(self, u, src, dst, c, cid, g):
            return c[px.WEIGHT, cid] * u[nets.GRAD_PRE_ACT, dst]

        def apply(self, u, i, g, acc):
            a = u[px.ACTIVATION, i]
            if name == "max":
                acc = jnp.maximum(acc, jnp.float32(-1.0))
            elif name == "min":
                acc = jnp.minimum(acc, jnp.float32(1.0))
            return px.UnitWrite.of((nets.GRAD_PRE_ACT, (acc + u[nets.LOSS_GRAD, i]) * (jnp.float32(1.0) - a * a)))

    Bwd.__name__ = f"Bwd_{name}"
    return Bwd()


def _kill(state, every: int = 7, units: tuple[int, ...] = ()) -> None:
    """Tombstones inside the rows (every `every`-th live slot) and every
    edge touching `units` (rows with no live term either way)."""
    for bucket in state.conns:
        live = torch.nonzero(bucket["dead"] == 0).flatten()
        bucket["dead"][live[::every]] = 1
        for u in units:
            bucket["dead"][(bucket["to_id"] == u) | (bucket["from_id"] == u)] = 1


def _zipf(net, scale: int, seed: int):
    e = synth.c2_topological(seed=seed, scale=scale)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cuda")
    width = e.input_ids.size
    rng = np.random.default_rng(seed + 100)

    def inputs(k):
        x = rng.standard_normal(width).astype(np.float32)
        return x, np.tanh(x[::-1]).astype(np.float32)

    return static, state, inputs, e


@pytest.mark.parametrize("name", list(MONOIDS))
def test_forward_monoid_on_a_zipf_net(oracle, name: str) -> None:
    """C2's generator at 1/256 width with the forward folding by max / min /
    prod, Adam, tombstones and two level-1 rows with no live in-edge."""
    net = nets.make_trained_net(f"MF_{name}", _forward(name), nets.TanhBackward(),
                                px.optim.adam(1e-3, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state, inputs, e = _zipf(net, 256, 31)
    w = e.input_ids.size
    _kill(state, 7, (w + 3, w + 77))
    print(f"forward {name}: {e.src.size} edges", flush=True)
    _run_both(net, static, state, oracle, inputs, 4, {1, 4})


@pytest.mark.parametrize("name", list(MONOIDS))
@pytest.mark.parametrize("tile,nsuper", [(None, None), (64, 5), (1024, 512)])
def test_backward_monoid_on_a_zipf_net(oracle, name: str, tile, nsuper) -> None:
    """The backward folding by max / min / prod over the tiled layout: the
    default tiling, and small tiles whose Zipf head lands in the hot running
    sums and whose tail in the cold partials; tombstones and rows with no
    live out-edge."""
    net = nets.make_trained_net(f"MB_{name}", nets.TanhForward(), _backward(name),
                                px.optim.adam(1e-3, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state, inputs, e = _zipf(net, 128, 32)
    w = e.input_ids.size
    _kill(state, 5, (w + 1, 2 * w + 9))
    print(f"backward {name}: tile {tile} nsuper {nsuper}", flush=True)
    _run_both(net, static, state, oracle, inputs, 4, {1, 4}, tile=tile, nsuper=nsuper)


@pytest.mark.parametrize("name", list(MONOIDS))
def test_monoids_on_hub_groups(oracle, name: str) -> None:
    """Short rows under hub sources (fan-in 4-12, weights of magnitude near
    1, so products stay well inside the normal range), the monoid in both
    passes; a hub's (tile, source) group spans 15 or more ranks."""
    e = nets.hub_edges(7)
    rng = np.random.default_rng(3)
    w = (rng.choice([-1.0, 1.0], e.src.size) * rng.uniform(0.7, 1.4, e.src.size)).astype(np.float32)
    net = nets.make_trained_net(f"MH_{name}", _forward(name), _backward(name),
                                px.optim.adam(1e-3, nets.GRAD_PRE_ACT), px.Propagation.TOPOLOGICAL)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=w, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cuda")
    width, n_out = e.input_ids.size, e.output_ids.size
    rx = np.random.default_rng(4)

    def inputs(k):
        x = rx.standard_normal(width).astype(np.float32)
        return x, np.tanh(x[:n_out]).astype(np.float32)

    _run_both(net, static, state, oracle, inputs, 4, {1, 4}, tile=128, nsuper=3)


@pytest.mark.parametrize("fwd,bwd", [("max", "min"), ("prod", "max"), ("min", "prod")])
def test_monoids_on_a_pipeline_net(oracle, fwd: str, bwd: str) -> None:
    """C1's recurrent PIPELINE net with a named monoid in each pass."""
    e = synth.c1_pipeline(0)
    net = nets.make_trained_net(f"MP_{fwd}_{bwd}", _forward(fwd), _backward(bwd),
                                px.optim.sgd(1e-2, nets.GRAD_PRE_ACT), px.Propagation.PIPELINE)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cuda")
    _kill(state, 11)
    a = synth.c1_target(0)
    rng = np.random.default_rng(8)

    def inputs(k):
        x = rng.standard_normal(32).astype(np.float32)
        return x, (a @ x).astype(np.float32)

    _run_both(net, static, state, oracle, inputs, 6, {1, 6})


@pytest.mark.parametrize("name", list(MONOIDS))
def test_batched_wide_levels_with_each_monoid(oracle, name: str) -> None:
    """Batched steps (B = 256) whose 384- and 320-row levels take the
    one-wave-per-row kernels, the monoid in both passes, skip edges
    carrying accumulators across levels."""
    from test_gpu_batched import _run

    opt = px.optim.adam(1e-3, nets.GRAD_PRE_ACT)

    class Net(px.Network):
        forward_pass = _forward(name)
        backward_pass = _backward(name)
        loss = nets.MSELoss()
        update_conn = opt.update_conn()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        extra_conn_fields = tuple(opt.state_fields)
        batch_reduction = px.MeanFloatFirstRest()

    _run(oracle, Net, [64, 384, 320, 8], 0.2, 0.02, 256, 2, seed=10 + len(name))


@pytest.mark.parametrize("pipeline", [False, True])
def test_generic_min_prod_max_tuple(oracle, pipeline: bool) -> None:
    """A generic forward with (min, prod, max) components over a varied
    UTIL column (signed powers of two), through plx_gen_fold; tombstones and
    a row with no live in-edge (components at +inf, 1, -inf)."""
    net = gc.make_net(gc.MinProdMaxForward(), nets.TanhBackward(), pipeline=pipeline,
                      optimizer=px.optim.adam(1e-2, nets.GRAD_PRE_ACT))
    static, state = gc.build(net, pipeline=pipeline, seed=21, device="cuda")
    rng = np.random.default_rng(22)
    for bucket in state.conns:
        n = bucket["dead"].numel()
        u = rng.choice([-1.0, 1.0], n) * np.exp2(rng.integers(-2, 3, n))
        bucket[gc.UTIL.name].copy_(torch.from_numpy(u.astype(np.float32)))
    _kill(state, 9, (30,))
    o = nets.oracle_for(oracle, net, static, state)
    step = px.make_step(net, static)
    if step.backward_order == "slot":
        o.tile = None
    xs, ts = gc.data(23, 4, len(static.input_ids), len(static.output_ids))
    for k in range(4):
        print(f"generic (min, prod, max) step {k} pipeline={pipeline}", flush=True)
        res = step(state, px.StepInputs(xs[k], ts[k]))
        state = res.state
        lo = o.step(xs[k], ts[k])
        torch.cuda.synchronize()
        assert_same_state(static, state, o, f"step {k}")
        assert _equal(np.float32([float(res.loss)]), np.float32([lo])), f"loss at step {k}"
    if not pipeline:
        assert o.units[gc.MN.name][30] == np.inf and o.units[gc.PR.name][30] == 1.0
