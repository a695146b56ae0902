"""Device structural phases against the CPU oracle, bit for bit.

Every growth golden case runs through the device pipeline
(plastax_amd.grow.AddConnPhase) and must commit exactly the reference's
edges and flags; the device's whole logical arena after the phase must equal
the oracle's (every column, every slot). Larger random cases (thousands of
units, tens of thousands of candidates, both propagation modes, every
candidate producer) compare device and oracle the same way, and the building
blocks (ordered compaction, scan, radix sort) are checked against numpy.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

import growth_cases as gc
import plastax_amd as px
import plastax_amd.numpy as jnp
from oracle import growth as og
from plastax_amd import _lib, grow
from plastax_amd.state import column_to_numpy, to_column

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _kernels() -> grow.Kernels:
    return grow.Kernels(DEV, torch.cuda.current_stream(DEV).cuda_stream)


def _to_device(hn: gc.HostNet) -> tuple[dict, tuple]:
    uspecs = {s.name: s for s in hn.static.unit_fields}
    cspecs = {s.name: s for s in hn.static.conn_fields}
    units = {k: to_column(v, uspecs[k], DEV) for k, v in hn.units.items()}
    conns = tuple({k: to_column(v, cspecs[k], DEV) for k, v in b.items()} for b in hn.conns)
    return units, conns


def _to_host(hn: gc.HostNet, conns: tuple) -> list[dict]:
    cspecs = {s.name: s for s in hn.static.conn_fields}
    return [{k: column_to_numpy(v, cspecs[k]) for k, v in b.items()} for b in conns]


def _device_grow(hn: gc.HostNet) -> tuple[grow.GrowthOutcome, list[dict]]:
    print(f"device growth: {type(hn.net.add_conn).__name__} units={hn.static.num_units} "
          f"caps={hn.static.level_capacities}", flush=True)
    units, conns = _to_device(hn)
    phase = grow.AddConnPhase(hn.net, hn.static, hn.globals_)
    out = phase.run(_kernels(), units, conns, step=hn.step, globals_=hn.globals_, tail_start=hn.tail_start,
                    units_added=hn.units_added)
    torch.cuda.synchronize()
    return out, _to_host(hn, out.conns)


def _oracle_grow(hn: gc.HostNet) -> og.GrowthResult:
    return og.add_conn(hn.net, hn.static, hn.units, hn.conns, step=hn.step, globals_=hn.globals_,
                       tail_start=hn.tail_start, units_added=hn.units_added)


def _same_arena(dev: list[dict], ref: list[dict]) -> None:
    assert len(dev) == len(ref)
    for b, (d, r) in enumerate(zip(dev, ref)):
        assert d.keys() == r.keys()
        for name in d:
            a, e = np.asarray(d[name]), np.asarray(r[name])
            if a.dtype.kind == "f":
                assert np.array_equal(a.view(np.uint32), e.astype(a.dtype).view(np.uint32)), (b, name)
            else:
                assert np.array_equal(a.astype(np.int64), e.astype(np.int64)), (b, name)


def _check(hn: gc.HostNet) -> tuple[grow.GrowthOutcome, list[dict]]:
    out, dev = _device_grow(hn)
    ref = _oracle_grow(hn)
    assert (out.grown, out.overflow, out.needs_resort, out.tail_start) == (
        ref.grown, ref.overflow, ref.needs_resort, ref.tail_start)
    _same_arena(dev, ref.conns)
    return out, dev


# ---------------------------------------------------------------------------
# Building blocks.
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("n", [1, 100, 2048, 5000, 70001])
def test_compact_and_scan(n: int) -> None:
    rng = np.random.default_rng(n)
    k = _kernels()
    flags = torch.from_numpy((rng.random(n) < 0.3).astype(np.uint8)).to(DEV)
    out, count = k.compact(n, 0, flags)
    want = np.flatnonzero(flags.cpu().numpy())
    assert int(count.item()) == want.size
    assert np.array_equal(out[: want.size].cpu().numpy(), want)
    vals = torch.from_numpy(rng.integers(0, 5, n).astype(np.int32)).to(DEV)
    res = torch.empty(n, dtype=torch.int32, device=DEV)
    total = torch.empty(1, dtype=torch.int32, device=DEV)
    scratch = k.mem.ints_for(n)
    _lib.check(k.lib.plx_scan_i32(n, None, vals.data_ptr(), res.data_ptr(), total.data_ptr(), scratch.data_ptr(),
                                  k.s), "scan")
    v = vals.cpu().numpy().astype(np.int64)
    assert np.array_equal(res.cpu().numpy(), np.concatenate([[0], np.cumsum(v)[:-1]]))
    assert int(total.item()) == int(v.sum())


@pytest.mark.parametrize("n", [1, 700, 1024, 1025, 4095, 4097, 100000])
def test_radix_sort_is_the_total_order(n: int) -> None:
    """(-score, src, dst, index) with ties, NaN, +-0 and +-inf, against
    numpy's lexsort (the oracle's total_order); up to 1,024 elements the
    one-workgroup sort, beyond it the radix passes."""
    rng = np.random.default_rng(n + 7)
    k = _kernels()
    score = rng.choice(np.array([0.5, -0.0, 0.0, np.inf, -np.inf, np.nan, 1.25, -3.0], np.float32), n)
    score = np.where(rng.random(n) < 0.5, rng.standard_normal(n).astype(np.float32), score).astype(np.float32)
    src = rng.integers(0, 300, n).astype(np.int32)
    dst = rng.integers(0, 70000, n).astype(np.int32)
    s_t, src_t, dst_t = (torch.from_numpy(a).to(DEV) for a in (score, src, dst))
    order = k.iota(n)
    k.sort(order, n, [(0, 17, dst_t, None), (0, 9, src_t, None), (1, 32, s_t, None)])
    assert np.array_equal(order[:n].cpu().numpy(), og.total_order(score, src, dst))


def test_small_sort_with_device_counts() -> None:
    """The one-workgroup sort (at most 1,024 elements) with a device count:
    the first count elements are sorted stably, the rest of the list is left
    as it was; with a count of 0 nothing is read (the entries past the count
    here are far outside the key column)."""
    k = _kernels()
    rng = np.random.default_rng(3)
    n_max = 900
    keys_np = rng.integers(0, 50, 5000).astype(np.int32)
    keys = torch.from_numpy(keys_np).to(DEV)
    base = rng.permutation(5000)[:n_max].astype(np.int32)
    for cnt in (0, 1, 517, n_max):
        v = base.copy()
        v[cnt:] = 2_000_000_000
        vt = torch.from_numpy(v).to(DEV)
        nd = torch.tensor([cnt], dtype=torch.int32, device=DEV)
        k.sort(vt, n_max, [(0, 6, keys, None)], n_dev=nd)
        got = vt.cpu().numpy()
        head = v[:cnt]
        assert np.array_equal(got[:cnt], head[np.argsort(keys_np[head], kind="stable")]), f"count {cnt}"
        assert np.array_equal(got[cnt:], v[cnt:]), f"count {cnt}: past the count"


# ---------------------------------------------------------------------------
# The reference's growth goldens on the device.
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("name", gc.PROPOSE_CASES)
def test_propose_golden_on_device(name: str) -> None:
    doc = gc.load(name)
    hn = gc.propose_net(doc)
    out, dev = _check(hn)
    assert gc.grown_pairs(hn.conns, dev) == gc.want_commits(doc["expect"])
    assert out.needs_resort == doc["expect"]["needs_resort"]


@pytest.mark.parametrize("name", gc.SCORE_CASES)
def test_score_golden_on_device(name: str) -> None:
    doc = gc.load(name)
    free_slots = int(doc["params"]["free_slots"])
    hn = gc.score_net(doc, step_cap=free_slots, free_at={})
    out, dev = _check(hn)
    assert gc.grown_pairs(hn.conns, dev) == gc.want_commits(doc["expect"])
    assert out.needs_resort == doc["expect"]["needs_resort"]
    _check(gc.score_net(doc, step_cap=None, free_at={}))


@pytest.mark.parametrize("name", gc.CLAIM_TOPO_CASES)
def test_claim_topological_golden_on_device(name: str) -> None:
    doc = gc.load(name)
    free = {int(k): v for k, v in doc["params"]["free_per_level"].items()}
    hn = gc.score_net(doc, step_cap=None, free_at=free)
    out, dev = _check(hn)
    assert gc.grown_pairs(hn.conns, dev) == gc.want_commits(doc["expect"])
    assert out.overflow == doc["expect"]["conn_overflow"]


@pytest.mark.parametrize("name", gc.CLAIM_PIPE_CASES)
def test_claim_pipeline_golden_on_device(name: str) -> None:
    doc = gc.load(name)
    hn = gc.pipeline_net(doc)
    out, dev = _check(hn)
    assert gc.grown_pairs(hn.conns, dev) == gc.want_commits(doc["expect"])
    assert out.tail_start - hn.tail_start == doc["expect"]["tail_used"]


# ---------------------------------------------------------------------------
# Larger random nets: device == oracle.
# ---------------------------------------------------------------------------


class _Relu(px.ForwardPass):
    combine = px.monoid.sum_

    def map(self, u, dst, src, c, cid, g):
        return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, jnp.maximum(acc, jnp.float32(0.0))))


def _random_net(rule, *, seed: int, n: int, levels: int, edges: int, pipeline: bool, dead_frac: float,
                with_capacity: bool = False) -> gc.HostNet:
    rng = np.random.default_rng(seed)
    mode = px.Propagation.PIPELINE if pipeline else px.Propagation.TOPOLOGICAL

    class Net(px.Network):
        forward_pass = _Relu()
        add_conn = rule
        propagation = mode
        extra_conn_fields = (px.FieldSpec.float32("trace", 0.25), px.FieldSpec.int32("age", 3))
        unit_capacity = n if with_capacity else None

    per = n // levels
    lvl = np.arange(n) // per
    lvl = np.minimum(lvl, levels - 1)
    if pipeline:
        src = rng.integers(0, n, edges)
        dst = rng.integers(0, n, edges)
    else:
        src = rng.integers(0, per * (levels - 1), edges)
        dst = np.minimum(lvl[src] + 1, levels - 1) * per + rng.integers(0, per, edges)
    w = (rng.integers(-8, 8, edges) / 8).astype(np.float32)
    n_built = n - (n // 10 if with_capacity else 0)
    keep = (src < n_built) & (dst < n_built)
    static, state = px.NetworkBuilder.from_edges(
        Net, n_built, src[keep].astype(np.int32), dst[keep].astype(np.int32), weights=w[keep],
        input_ids=list(range(min(4, per))), output_ids=[n_built - 1], globals_={"thr": np.float32(0.1)},
        capacity_headroom=0.5, device="cpu")
    hn_units, hn_conns = gc._host(state, static)
    hn_units["activation"] = rng.standard_normal(hn_units["activation"].shape[0]).astype(np.float32)
    conns = []
    for b in hn_conns:
        b = {k2: v.copy() for k2, v in b.items()}
        live = np.flatnonzero(~b["dead"].astype(bool))
        kill = live[rng.random(live.size) < dead_frac]
        b["dead"][kill] = True
        conns.append(b)
    tail = int(state.tail_start)
    return gc.HostNet(Net, static, hn_units, conns, {"thr": np.float32(0.1)}, step=17 + seed, tail_start=tail)


def _propose(kind: str, n: int, *, P: int, k: int, gap: int, ded_live: bool, ded_step: bool, **knobs):
    class Rule(px.ProposeAddConn):
        proposer = kind
        proposals_per_proposer = P
        max_new_per_level = k
        max_level_gap = gap
        dedupe_live = ded_live
        dedupe_step = ded_step

        def propose(self, *args):
            if kind == "per_unit":
                u, i, j, g, rng = args
                src = jnp.asarray(i, jnp.int32)
            elif kind == "per_connection":
                u, c, cid, j, g, rng = args
                src = jnp.where(rng.bernoulli(0.5), c[px.TO_ID, cid], c[px.FROM_ID, cid])
            else:
                u, j, g, rng = args
                src = rng.uniform_int(n).astype(jnp.int32)
            dst = rng.uniform_int(n).astype(jnp.int32)
            act = u[px.ACTIVATION, dst]
            return src, dst, jnp.floor(rng.uniform() * jnp.float32(64.0)) + act * jnp.float32(0.0)

        def init(self, u, src, dst, g):
            return px.ConnWrite.of((px.WEIGHT, u[px.ACTIVATION, src] * jnp.float32(0.5)),
                                   (px.FieldSpec.int32("age", 3), (src * 7 + dst) % 5))

    for key, v in knobs.items():
        setattr(Rule, key, v)
    return Rule()


@pytest.mark.parametrize("seed", [0, 1])
@pytest.mark.parametrize("kind", ["per_unit", "per_connection", "global"])
@pytest.mark.parametrize("pipeline", [False, True])
def test_random_propose_matches_oracle(seed: int, kind: str, pipeline: bool) -> None:
    n = 3000
    rule = _propose(kind, n, P=4 if kind != "global" else 5000, k=40, gap=3 if pipeline else 1,
                    ded_live=bool(seed), ded_step=True, direction="any" if pipeline else "deeper")
    hn = _random_net(rule, seed=seed, n=n, levels=4, edges=12000, pipeline=pipeline, dead_frac=0.05,
                     with_capacity=bool(seed))
    out, _ = _check(hn)
    assert out.grown > 0


def test_normal_draws_in_proposals_match_oracle() -> None:
    """Per-unit proposals scored by Rng.normal (Box-Muller on two uniforms,
    rng.py:289-299: Cephes log and cos on both sides) and a normal draw mixed
    into the destination: the commits and every column, bit for bit."""
    n = 3000

    class NormalRule(px.ProposeAddConn):
        proposer = "per_unit"
        proposals_per_proposer = 4
        max_new_per_level = 40
        max_level_gap = 3
        direction = "any"
        dedupe_step = True

        def propose(self, u, i, j, g, rng):
            z = rng.normal()
            dst = (jnp.abs(z) * jnp.float32(700.0)).astype(jnp.int32) % n
            return jnp.asarray(i, jnp.int32), dst, rng.normal() + jnp.cos(u[px.ACTIVATION, i])

        def init(self, u, src, dst, g):
            return px.ConnWrite.of((px.WEIGHT, jnp.sin(u[px.ACTIVATION, src]) * jnp.float32(0.5)))

    hn = _random_net(NormalRule(), seed=5, n=n, levels=4, edges=12000, pipeline=True, dead_frac=0.05,
                     with_capacity=False)
    out, _ = _check(hn)
    assert out.grown > 0


def _score_rule(cands: str, *, k: int | None, M: int, **knobs):
    class Rule(px.ScoreAddConn):
        candidates = cands
        shortlist_size = M
        max_new_per_level = k

        def score(self, u, src, dst, g):
            return jnp.abs(u[px.ACTIVATION, src] - u[px.ACTIVATION, dst]) + ((src + dst) % 3).astype(jnp.float32)

        def importance(self, u, i, g):
            return jnp.abs(u[px.ACTIVATION, i])

        def threshold(self, g):
            return g["thr"]

        def init(self, u, src, dst, g):
            return px.ConnWrite.of((px.WEIGHT, jnp.float32(0.125)))

    for key, v in knobs.items():
        setattr(Rule, key, v)
    return Rule()


@pytest.mark.parametrize("case", [
    dict(cands="shortlist_per_level", k=30, M=24, direction="deeper", dedupe_live=True),
    dict(cands="shortlist_per_level", k=30, M=24, level_cap_scope="step", max_new_per_step=50),
    dict(cands="shortlist", k=25, M=40, selection="threshold", max_level_gap=2),
    dict(cands="exhaustive", k=20, M=0, dedupe_step=True, allow_self_loops=True),
])
def test_random_score_matches_oracle(case: dict) -> None:
    knobs = dict(case)
    rule = _score_rule(knobs.pop("cands"), k=knobs.pop("k"), M=knobs.pop("M"), **knobs)
    n = 240 if rule.candidates == "exhaustive" else 3000
    hn = _random_net(rule, seed=3, n=n, levels=4, edges=4 * n, pipeline=False, dead_frac=0.1)
    out, _ = _check(hn)
    assert out.grown > 0


def test_random_score_pipeline_matches_oracle() -> None:
    rule = _score_rule("shortlist", k=5, M=60, max_level_gap=50)
    hn = _random_net(rule, seed=5, n=2000, levels=6, edges=6000, pipeline=True, dead_frac=0.2)
    _check(hn)


# ---------------------------------------------------------------------------
# PruneConn.
# ---------------------------------------------------------------------------


def test_prune_conn_matches_oracle() -> None:
    class Prune(px.PruneConn):
        def predicate(self, u, c, cid, g):
            w = c[px.WEIGHT, cid]
            return (jnp.abs(w) < g["thr"]) | (u[px.ACTIVATION, c[px.FROM_ID, cid]] > jnp.float32(1.5))

    rule = _propose("per_unit", 3000, P=1, k=1, gap=1, ded_live=False, ded_step=False)
    hn = _random_net(rule, seed=9, n=3000, levels=4, edges=12000, pipeline=False, dead_frac=0.0)

    class Net(hn.net):
        prune_conn = Prune()

    units, conns = _to_device(hn)
    phase = grow.PruneConnPhase(Net, hn.static, hn.globals_)
    phase.run(_kernels(), units, conns, hn.globals_)
    dev = _to_host(hn, conns)
    prog = phase.prog
    ref = og.prune_conn(prog, hn.units, hn.conns, hn.globals_)
    _same_arena(dev, ref)
    assert sum(int(b["dead"].sum()) for b in dev) > sum(int(b["dead"].sum()) for b in hn.conns)
