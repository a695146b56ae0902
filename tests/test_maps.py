"""Product maps: (connection factor) * (unit factor at the other end), either
factor WEIGHT / a field or a float constant, or a lone factor (the reference
runs any map, sweep.py:113-180; the device runs this family,
_expr.product_map). CPU: the tracer's classification, and the oracle pinned by
closed forms -- a constant map under sum_ counts live in-edges (forward) and
out-edges (backward), a weight-only map sums a unit's in-weights."""

from __future__ import annotations

import numpy as np
import pytest

import nets
import plastax_amd as px
import plastax_amd.numpy as jnp
from plastax_amd._expr import Index, TraceConnView, TraceUnitView, UnsupportedPolicyError, product_map

INDEG = px.FieldSpec.float32("indeg")
OUTDEG = px.FieldSpec.float32("outdeg")
WSUM = px.FieldSpec.float32("wsum")


def _views():
    u = TraceUnitView({"activation": np.float32, "g": np.float32})
    c = TraceConnView({"weight": np.float32, "dead": np.bool_})
    return u, c


@pytest.mark.parametrize("make,want", [
    (lambda u, c: c[px.WEIGHT, Index("cid")] * u[px.ACTIVATION, Index("src")], ("activation", None, None)),
    (lambda u, c: u[px.ACTIVATION, Index("src")] * c[px.WEIGHT, Index("cid")], ("activation", None, None)),
    (lambda u, c: jnp.float32(1.0), (None, 1.0, 1.0)),
    (lambda u, c: 2.5, (None, 2.5, 1.0)),
    (lambda u, c: u[px.ACTIVATION, Index("src")], ("activation", 1.0, None)),
    (lambda u, c: c[px.WEIGHT, Index("cid")], (None, None, 1.0)),
    (lambda u, c: jnp.float32(0.5) * u[px.ACTIVATION, Index("src")], ("activation", 0.5, None)),
    (lambda u, c: c[px.WEIGHT, Index("cid")] * 3.0, (None, None, 3.0)),
    (lambda u, c: jnp.float32(2.0) * jnp.float32(3.0), (None, 6.0, 1.0)),
])
def test_product_map_factors(make, want) -> None:
    u, c = _views()
    pm = product_map(make(u, c), "src")
    got = (pm.field, None if pm.w_const is None else float(pm.w_const),
           None if pm.x_const is None else float(pm.x_const))
    assert got == want


@pytest.mark.parametrize("make", [
    lambda u, c: c[px.WEIGHT, Index("cid")] * c[px.WEIGHT, Index("cid")],
    lambda u, c: u[px.ACTIVATION, Index("dst")] * c[px.WEIGHT, Index("cid")],  # the wrong end
    lambda u, c: c[px.WEIGHT, Index("cid")] * u[px.ACTIVATION, Index("src")] * 2.0,  # three factors
    lambda u, c: c[px.WEIGHT, Index("cid")] + u[px.ACTIVATION, Index("src")],
])
def test_other_maps_are_refused(make) -> None:
    u, c = _views()
    with pytest.raises(UnsupportedPolicyError):
        product_map(make(u, c), "src")


class CountIn(px.ForwardPass):
    combine = px.monoid.sum_

    def map(self, u, dst, src, c, cid, g):
        return jnp.float32(1.0)

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((INDEG, acc))


class WeightSum(px.ForwardPass):
    combine = px.monoid.sum_

    def map(self, u, dst, src, c, cid, g):
        return c[px.WEIGHT, cid]

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((WSUM, acc))


class CountOut(px.BackwardPass):
    combine = px.monoid.sum_

    def map(self, u, src, dst, c, cid, g):
        return jnp.float32(1.0)

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((OUTDEG, acc))


def degree_net(forward, propagation):
    return type("DegreeNet", (px.Network,), dict(
        forward_pass=forward, backward_pass=CountOut(), extra_unit_fields=(INDEG, OUTDEG, WSUM),
        propagation=propagation))


@pytest.mark.parametrize("pipeline", [False, True])
def test_oracle_counts_and_sums_match_closed_forms(oracle, pipeline: bool) -> None:
    """One step of the oracle: indeg / outdeg are the live in- and out-edge
    counts of every finalized unit, exactly; the weight sum of a unit whose
    in-weights are dyadic (exact in any order) is their sum."""
    rng = np.random.default_rng(4)
    if pipeline:
        n = 300
        src = rng.integers(0, n, 2000).astype(np.int32)
        dst = rng.integers(0, n, 2000).astype(np.int32)
        keep = src != dst
        src, dst = src[keep], dst[keep]
        ins, outs = np.arange(8), np.arange(n - 4, n)
    else:
        e = nets.hub_edges(3)
        n, src, dst, ins, outs = e.num_units, e.src, e.dst, e.input_ids, e.output_ids
    w = (rng.integers(-64, 64, src.size) / 16.0).astype(np.float32)
    for fwd, col in ((CountIn(), "indeg"), (WeightSum(), "wsum")):
        net = degree_net(fwd, px.Propagation.PIPELINE if pipeline else px.Propagation.TOPOLOGICAL)
        static, state = px.NetworkBuilder.from_edges(
            net, n, src, dst, weights=w, input_ids=ins, output_ids=outs, globals_=None, device="cpu")
        o = nets.oracle_for(oracle, net, static, state)
        o.tile = None
        o.step(np.zeros(len(ins), np.float32))
        non_input = np.ones(n, bool)
        non_input[ins] = False
        if col == "indeg":
            want = np.bincount(dst, minlength=n).astype(np.float32)
        else:
            want = np.zeros(n, np.float64)
            np.add.at(want, dst, w.astype(np.float64))
            want = want.astype(np.float32)
        assert np.array_equal(o.units[col][non_input], want[non_input])
        outdeg = np.bincount(src, minlength=n).astype(np.float32)
        has_level = non_input if pipeline else np.ones(n, bool)
        if not pipeline:
            # a TOPOLOGICAL backward finalizes levels 1..L (inputs at level 0 keep their default)
            has_level = o.units["level"] > 0
        assert np.array_equal(o.units["outdeg"][has_level & non_input], outdeg[has_level & non_input])
