"""BASELINE config C5's recipe as a plastax network: a growing PIPELINE
reservoir (tanh), a backward pass that counts every unit's live out-edges
(a constant map under sum_), PruneUnit of the units whose out-degree is
zero, AddUnit spawning a fixed band of parents every `every` steps (a global
flag the driver raises), and ProposeAddConn per unit with P = 4 proposals
drawn from the counter-based rng."""

from __future__ import annotations

import numpy as np

import plastax_amd as px
import plastax_amd.numpy as jnp

OUTDEG = px.FieldSpec.float32("out_degree")


class TanhReservoir(px.ForwardPass):
    combine = px.monoid.sum_

    def map(self, u, dst, src, c, cid, g):
        return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)))


class CountOutEdges(px.BackwardPass):
    combine = px.monoid.sum_

    def map(self, u, src, dst, c, cid, g):
        return jnp.float32(1.0)

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((OUTDEG, acc))


class PruneSilent(px.PruneUnit):
    def predicate(self, u, i, g):
        return u[OUTDEG, i] == jnp.float32(0.0)


def recipe(num_inputs: int, num_targets: int, spawn_lo: int, spawn_n: int, max_new: int,
           unit_capacity: int) -> type:
    """The C5 network class: proposals target ids below ``num_targets``;
    the parents with ids in [spawn_lo, spawn_lo + spawn_n) spawn when the
    global ``spawn`` is set."""
    cap = unit_capacity

    class SpawnBand(px.AddUnit):
        def spawn(self, u, parent, g):
            band = (parent >= spawn_lo) & (parent < spawn_lo + spawn_n)
            return band & (g["spawn"] > jnp.float32(0.0)), jnp.int32(0)

        def init(self, u, child, parent, g):
            return px.UnitWrite.of((px.ACTIVATION, u[px.ACTIVATION, parent] * jnp.float32(0.5)))

    class ProposePerUnit(px.ProposeAddConn):
        proposer = "per_unit"
        proposals_per_proposer = 4
        max_new_per_level = max_new
        max_level_gap = 1 << 20

        def propose(self, u, i, j, g, rng):
            dst = rng.uniform_int(num_targets).astype(jnp.int32)
            return jnp.asarray(i, jnp.int32), dst, rng.uniform()

        def init(self, u, src, dst, g):
            return px.ConnWrite.of((px.WEIGHT, jnp.float32(0.01)))

    class C5Reservoir(px.Network):
        unit_capacity = cap
        forward_pass = TanhReservoir()
        backward_pass = CountOutEdges()
        prune_unit = PruneSilent()
        add_unit = SpawnBand()
        add_conn = ProposePerUnit()
        extra_unit_fields = (OUTDEG,)
        propagation = px.Propagation.PIPELINE

    return C5Reservoir


def reservoir_edges(seed: int, n: int, edges: int, num_inputs: int) -> tuple[np.ndarray, ...]:
    """Random recurrent edges (no self-loops) whose weights are N(0, 1)
    scaled to a spectral radius of about 0.9 (1 / sqrt(n * density))."""
    rng = np.random.default_rng(seed)
    src = rng.integers(0, n, edges).astype(np.int32)
    dst = rng.integers(num_inputs, n, edges).astype(np.int32)
    keep = src != dst
    src, dst = src[keep], dst[keep]
    scale = 0.9 / np.sqrt(src.size / n)
    w = (rng.standard_normal(src.size) * scale).astype(np.float32)
    return src, dst, w
