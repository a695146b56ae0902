"""The oracle's named-monoid folds -- ``max_``, ``min_`` and ``prod`` -- pinned
against numpy's scatter ufuncs (``np.maximum.at``, ``np.minimum.at``,
``np.multiply.at``), an independent implementation of the same segment reduce
(``jax.ops.segment_max / segment_min / segment_prod``, monoid.py:29-51,
:84-122) and of ``combine_pairwise`` (``jnp.maximum / minimum / multiply``,
monoid.py:46-51, :124-152).

What the checks fix, each chosen so that a plausible mistake fails:

- the identity of a segment with no live term: -inf, +inf, 1.0 (a wrong
  identity, or a dead slot entering the fold, changes those rows);
- NaN propagation: a NaN term makes its segment NaN, wherever it sits in the
  fold (a C ``fmaxf`` would drop it);
- ties of equal value: ``a > b ? a : b`` keeps the later operand, which only
  shows between -0.0 and +0.0 (numpy's ufuncs behave the same way; XLA's
  signed-zero tie rule cannot be run here and is parity unpinned);
- the fold order of the tiled backward (tiles, superblocks, runs): products of
  dyadic values are exact, so ``np.multiply.at`` in the fold's order must give
  the same bits; max / min pick the same element under any grouping of one
  order;
- the level walk: a bucket's segment result combined into the carried
  accumulator, skip edges, finalization by level (whole-net tests).

Every comparison is bit for bit, except that two NaNs compare equal (their
payloads depend on which operand the compiler placed first).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import generic_cases as gc
import nets
import plastax_amd as px
import plastax_amd.numpy as jnp

MONOIDS = {
    "max": (px.monoid.max_, np.maximum, -np.inf),
    "min": (px.monoid.min_, np.minimum, np.inf),
    "prod": (px.monoid.prod, np.multiply, 1.0),
}
_i64p = ctypes.POINTER(ctypes.c_int64)
NAN = np.float32(np.nan)


def _same(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    if a.shape != b.shape:
        return False
    both_nan = np.isnan(a) & np.isnan(b)
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | both_nan))


def _diff(a: np.ndarray, b: np.ndarray) -> str:
    bad = np.flatnonzero((a.view(np.uint32) != b.view(np.uint32)) & ~(np.isnan(a) & np.isnan(b)))
    return f"{bad.size} differ; first at {bad[:1]}: oracle {a[bad[:1]]} numpy {b[bad[:1]]}"


def _dyadic(rng: np.random.Generator, n: int, zeros: float = 0.08) -> np.ndarray:
    """Signed powers of two in [2^-3, 2^3], with a share of +0.0 and -0.0."""
    v = (rng.choice([-1.0, 1.0], n) * np.exp2(rng.integers(-3, 4, n))).astype(np.float32)
    z = rng.random(n) < zeros
    v[z] = np.where(rng.random(int(z.sum())) < 0.5, np.float32(0.0), np.float32(-0.0))
    return v


class _Bucket:
    """A bucket of `cap` slots over `n` units. Units 40..47 are endpoints of
    dead slots only and 48..63 of no slot, so they are rows with no live term
    in both directions; a quarter of the other slots are dead too (inside
    rows). Weights and unit values are dyadic with signed zeros; unit 7's
    value is NaN when `nan` is set."""

    def __init__(self, seed: int, nan: bool, cap: int = 700, n: int = 64) -> None:
        rng = np.random.default_rng(seed)
        self.n = n
        self.cap = cap
        self.from_id = rng.integers(0, 48, cap).astype(np.int32)
        self.to_id = rng.integers(0, 48, cap).astype(np.int32)
        dead = rng.random(cap) < 0.25
        dead |= (self.from_id >= 40) | (self.to_id >= 40)
        self.dead = dead.astype(np.uint8)
        self.weight = _dyadic(rng, cap)
        self.x = _dyadic(rng, n)
        self.g = _dyadic(rng, n)
        if nan:
            self.x[7] = NAN
            self.g[7] = NAN
        self.live = np.flatnonzero(self.dead == 0)
        self.rng = rng

    def fwd_terms(self) -> np.ndarray:
        return (self.weight * self.x[self.from_id]).astype(np.float32)

    def bwd_terms(self) -> np.ndarray:
        return (self.weight * self.g[self.to_id]).astype(np.float32)


def _scatter(ufunc, ident: float, n: int, keys: np.ndarray, vals: np.ndarray) -> np.ndarray:
    out = np.full(n, ident, np.float32)
    with np.errstate(invalid="ignore"):
        ufunc.at(out, keys, vals)
    return out


@pytest.mark.parametrize("nan", [False, True])
@pytest.mark.parametrize("name", list(MONOIDS))
def test_forward_bucket_folds_match_numpy(oracle, name: str, nan: bool) -> None:
    """ox_bucket_reduce_fwd (slot order) and ox_bucket_reduce_fwd_rows (by
    destination rows) against a scatter of the live terms in slot order."""
    from oracle.oracle import bptr, fptr, iptr

    mono, ufunc, ident = MONOIDS[name]
    lib = oracle.load()
    code = mono.code
    assert lib.ox_identity(code) == np.float32(ident)
    for seed in range(6):
        b = _Bucket(seed, nan)
        want = _scatter(ufunc, ident, b.n, b.to_id[b.live], b.fwd_terms()[b.live])
        assert np.all(want[40:] == np.float32(ident))
        got = np.full(b.n, ident, np.float32)
        lib.ox_bucket_reduce_fwd(b.cap, iptr(b.from_id), iptr(b.to_id), bptr(b.dead), fptr(b.weight),
                                 fptr(b.x), code, fptr(got))
        assert _same(got, want), f"seed {seed} slot order: {_diff(got, want)}"
        # by rows: each destination's live slots ascending
        slots = b.live[np.argsort(b.to_id[b.live], kind="stable")].astype(np.int64)
        dst = b.to_id[slots]
        starts = np.concatenate([[0], np.flatnonzero(np.diff(dst)) + 1, [slots.size]]).astype(np.int64)
        units = np.ascontiguousarray(dst[starts[:-1]].astype(np.int32))
        got = np.full(b.n, ident, np.float32)
        lib.ox_bucket_reduce_fwd_rows(units.size, starts.ctypes.data_as(_i64p), slots.ctypes.data_as(_i64p),
                                      iptr(units), iptr(b.from_id), fptr(b.weight), fptr(b.x), code, fptr(got))
        assert _same(got, want), f"seed {seed} rows: {_diff(got, want)}"
        if nan:
            hit = np.unique(b.to_id[b.live][b.from_id[b.live] == 7])
            assert hit.size and np.all(np.isnan(got[hit]))


@pytest.mark.parametrize("nan", [False, True])
@pytest.mark.parametrize("name", list(MONOIDS))
def test_backward_bucket_folds_match_numpy(oracle, name: str, nan: bool) -> None:
    """ox_bucket_reduce_bwd (the slot-order fold, whole and in pieces of 3)
    against a scatter of the live terms into their sources in slot order."""
    from oracle.oracle import bptr, fptr, iptr

    mono, ufunc, ident = MONOIDS[name]
    lib = oracle.load()
    code = mono.code
    for seed in range(6):
        b = _Bucket(100 + seed, nan)
        want = _scatter(ufunc, ident, b.n, b.from_id[b.live], b.bwd_terms()[b.live])
        assert np.all(want[40:] == np.float32(ident))
        for piece in (1 << 30, 3):
            got = np.full(b.n, ident, np.float32)
            pc = np.zeros(b.n, np.float32)
            pn = np.zeros(b.n, np.int32)
            lib.ox_bucket_reduce_bwd(b.cap, iptr(b.from_id), iptr(b.to_id), bptr(b.dead), fptr(b.weight),
                                     fptr(b.g), b.n, code, piece, fptr(got), fptr(pc), iptr(pn))
            assert _same(got, want), f"seed {seed} piece {piece}: {_diff(got, want)}"


@pytest.mark.parametrize("nan", [False, True])
@pytest.mark.parametrize("name", list(MONOIDS))
def test_tiled_backward_folds_match_numpy(oracle, name: str, nan: bool) -> None:
    """ox_bucket_reduce_bwd_tiled and its parallel form by source runs, over
    the device's fold structure: per source, its terms in physical order
    (destinations renumbered by a permutation, then slot), grouped into
    tiles of 16 positions and superblocks of 3 tiles. The closed form
    scatters the same terms in that order; carried values in `out` (a
    previous bucket's result) are combined first, as in the walk."""
    from oracle.oracle import fptr, iptr

    mono, ufunc, ident = MONOIDS[name]
    lib = oracle.load()
    code = mono.code
    for seed in range(6):
        b = _Bucket(200 + seed, nan)
        phys = b.rng.permutation(b.n)
        live = b.live
        pos = np.empty(live.size, np.int64)
        pos[np.lexsort((live, phys[b.to_id[live]]))] = np.arange(live.size)
        tile = np.zeros(b.cap, np.int32)
        sb = np.zeros(b.cap, np.int32)
        tile[live] = pos // 16
        sb[live] = pos // 48
        order = np.ascontiguousarray(live[np.lexsort((live, phys[b.to_id[live]], b.from_id[live]))].astype(np.int64))
        carried = _dyadic(b.rng, b.n)
        carried[40:] = np.float32(ident)
        terms = b.bwd_terms()
        want = carried.copy()
        with np.errstate(invalid="ignore"):
            ufunc.at(want, b.from_id[order], terms[order])
        got = carried.copy()
        lib.ox_bucket_reduce_bwd_tiled(order.size, order.ctypes.data_as(_i64p), iptr(b.from_id), iptr(b.to_id),
                                       fptr(b.weight), fptr(b.g), iptr(tile), iptr(sb), code, fptr(got))
        assert _same(got, want), f"seed {seed} tiled: {_diff(got, want)}"
        fr = b.from_id[order]
        run_off = np.concatenate([[0], np.flatnonzero(np.diff(fr)) + 1, [order.size]]).astype(np.int64)
        got = carried.copy()
        lib.ox_bucket_reduce_bwd_tiled_runs(run_off.size - 1, run_off.ctypes.data_as(_i64p),
                                            order.ctypes.data_as(_i64p), iptr(b.from_id), iptr(b.to_id),
                                            fptr(b.weight), fptr(b.g), iptr(tile), iptr(sb), code, fptr(got))
        assert _same(got, want), f"seed {seed} runs: {_diff(got, want)}"


@pytest.mark.parametrize("name", list(MONOIDS))
def test_combine_pairwise_matches_numpy(oracle, name: str) -> None:
    """ox_combine against the elementwise ufunc, over every pair of special
    values in both orders (signed zeros, infinities, NaN, equal values)."""
    from oracle.oracle import fptr

    mono, ufunc, _ = MONOIDS[name]
    lib = oracle.load()
    sp = np.float32([0.0, -0.0, 1.0, -1.0, 0.5, -2.0, np.inf, -np.inf, np.nan, 3.0e38, 1e-45, -1e-45])
    a = np.repeat(sp, sp.size)
    b = np.tile(sp, sp.size)
    rng = np.random.default_rng(9)
    ra = _dyadic(rng, 4000)
    rb = _dyadic(rng, 4000)
    a = np.concatenate([a, ra]).astype(np.float32)
    b = np.concatenate([b, rb]).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        want = ufunc(a, b).astype(np.float32)
    got = a.copy()
    lib.ox_combine(a.size, mono.code, fptr(got), fptr(b))
    assert _same(got, want), _diff(got, want)
    if name != "prod":  # the tie rule: the later operand on equal values
        pz = np.float32([0.0, -0.0])
        got = pz.copy()
        lib.ox_combine(2, mono.code, fptr(got), fptr(pz[::-1].copy()))
        assert np.signbit(got).tolist() == [True, False]


# ---------------------------------------------------------------------------
# Whole walks: the named monoid through the level walk of the oracle.
# ---------------------------------------------------------------------------

RED = px.FieldSpec.float32("test/red")


def _forward_net(mono):
    class Fwd(px.ForwardPass):
        combine = mono

        def map(self, u, dst, src, c, cid, g):
            return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((px.ACTIVATION, acc))

    class Net(px.Network):
        forward_pass = Fwd()
        propagation = px.Propagation.TOPOLOGICAL

    return Net


def _backward_net(mono):
    class Bwd(px.BackwardPass):
        combine = mono

        def map(self, u, src, dst, c, cid, g):
            return c[px.WEIGHT, cid] * u[nets.GRAD_PRE_ACT, dst]

        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((nets.GRAD_PRE_ACT, acc + u[nets.LOSS_GRAD, i]))

    class Net(px.Network):
        forward_pass = nets.LinearForward()
        backward_pass = Bwd()
        extra_unit_fields = (nets.GRAD_PRE_ACT, nets.LOSS_GRAD)
        propagation = px.Propagation.TOPOLOGICAL

    return Net


def _layered(seed: int, rng_vals: np.random.Generator):
    """Four levels of 10 / 14 / 12 / 6 units, fan-in 3 plus skip edges from
    level 0 into level 2 (accumulators carried across buckets)."""
    rng = np.random.default_rng(seed)
    widths = [10, 14, 12, 6]
    base = np.concatenate([[0], np.cumsum(widths)])
    src, dst = [], []
    for l in range(3):
        for j in range(widths[l + 1]):
            for i in rng.choice(widths[l], 3, replace=False):
                src.append(base[l] + i)
                dst.append(base[l + 1] + j)
    for _ in range(8):
        src.append(int(rng.integers(0, widths[0])))
        dst.append(int(base[2] + rng.integers(0, widths[2])))
    src = np.asarray(src, np.int32)
    dst = np.asarray(dst, np.int32)
    w = (rng_vals.choice([-1.0, 1.0], src.size) * np.exp2(rng_vals.integers(-1, 2, src.size))).astype(np.float32)
    return int(base[-1]), src, dst, w, np.arange(widths[0]), np.arange(base[-2], base[-1])


def _kill(o, rng: np.random.Generator, unit: int = 12) -> None:
    """Tombstone a fifth of the live slots and every edge of `unit` (a
    level-1 row with no live term either way) in the oracle's logical
    arena."""
    for c in o.conns:
        live = np.flatnonzero(c["dead"] == 0)
        c["dead"][live[rng.random(live.size) < 0.2]] = 1
        c["dead"][(c["to_id"] == unit) | (c["from_id"] == unit)] = 1


@pytest.mark.parametrize("name", list(MONOIDS))
def test_forward_walk_matches_numpy_segment_reduce(oracle, name: str) -> None:
    """The oracle's TOPOLOGICAL forward with a named monoid and an identity
    apply equals the reference's walk written with numpy scatters:
    per bucket a fresh segment reduce of the live terms in slot order,
    combined into the carried accumulator, then level l+1 finalized."""
    mono, ufunc, ident = MONOIDS[name]
    rv = np.random.default_rng(5)
    n, src, dst, w, ins, outs = _layered(3, rv)
    net = _forward_net(mono)
    static, state = px.NetworkBuilder.from_edges(net, n, src, dst, weights=w, input_ids=ins, output_ids=outs,
                                                 globals_=None, capacity_headroom=0.25)
    o = nets.oracle_for(oracle, net, static, state)
    _kill(o, np.random.default_rng(7))
    x = _dyadic(rv, ins.size, zeros=0.2)
    o.units["activation"][ins] = x
    act = o.units["activation"].copy()
    levels = o.units["level"]
    is_in = np.zeros(n, bool)
    is_in[ins] = True
    acc = np.full(n, ident, np.float32)
    for lv, c in enumerate(o.conns):
        live = c["dead"] == 0
        seg = _scatter(ufunc, ident, n, c["to_id"][live], (c["weight"] * act[c["from_id"]])[live])
        with np.errstate(invalid="ignore"):
            acc = ufunc(acc, seg).astype(np.float32)
        fin = (levels == lv + 1) & ~is_in
        act[fin] = acc[fin]
    o.forward()
    assert _same(o.units["activation"], act), _diff(o.units["activation"], act)
    assert o.units["activation"][12] == np.float32(ident)  # no live in-edge: the identity


@pytest.mark.parametrize("name", list(MONOIDS))
def test_backward_walk_matches_numpy_segment_reduce(oracle, name: str) -> None:
    """The oracle's TOPOLOGICAL backward (the reference's slot-order fold)
    with a named monoid equals the numpy walk: the deepest level from the
    identity, then buckets L-1..1, each a fresh segment reduce into FROM_ID
    combined into the carried accumulator, level l finalized."""
    mono, ufunc, ident = MONOIDS[name]
    rv = np.random.default_rng(6)
    n, src, dst, w, ins, outs = _layered(4, rv)
    net = _backward_net(mono)
    static, state = px.NetworkBuilder.from_edges(net, n, src, dst, weights=w, input_ids=ins, output_ids=outs,
                                                 globals_=None, capacity_headroom=0.25)
    o = nets.oracle_for(oracle, net, static, state)
    o.tile = None
    _kill(o, np.random.default_rng(8))
    lg = np.zeros(n, np.float32)
    lg[outs] = _dyadic(rv, outs.size, zeros=0.0)
    o.units["loss_grad"][:] = lg
    levels = o.units["level"]
    is_in = np.zeros(n, bool)
    is_in[ins] = True
    nb = len(o.conns)
    grad = o.units["grad_pre_act"].copy()
    acc = np.full(n, ident, np.float32)
    top = (levels == nb) & ~is_in
    grad[top] = (acc + lg)[top]
    for lv in range(nb - 1, 0, -1):
        c = o.conns[lv]
        live = c["dead"] == 0
        seg = _scatter(ufunc, ident, n, c["from_id"][live], (c["weight"] * grad[c["to_id"]])[live])
        with np.errstate(invalid="ignore"):
            acc = ufunc(acc, seg).astype(np.float32)
        fin = (levels == lv) & ~is_in
        grad[fin] = (acc + lg)[fin]
    o.backward()
    assert _same(o.units["grad_pre_act"], grad), _diff(o.units["grad_pre_act"], grad)
    assert o.units["grad_pre_act"][12] == np.float32(ident)  # no live out-edge: the identity


def test_generic_tuple_components_match_numpy(oracle) -> None:
    """A generic forward with (min, prod, max) components: each component
    equals its numpy scatter over the live in-edges, with empty rows at the
    identities and a NaN term propagating in the max component."""
    net = gc.make_net(gc.MinProdMaxForward(), nets.TanhBackward())
    static, state = gc.build(net, pipeline=False, seed=5)
    o = nets.oracle_for(oracle, net, static, state)
    o.tile = None
    rng = np.random.default_rng(1)
    n = static.num_units
    _kill(o, rng, unit=30)  # a level-1 unit of the 24-60-50-8 net
    for c in o.conns:
        c[gc.UTIL.name] = _dyadic(rng, c["dead"].size)
    c0 = o.conns[1]
    nan_slot = np.flatnonzero(c0["dead"] == 0)[3]
    c0[gc.UTIL.name][nan_slot] = NAN
    x = rng.standard_normal(len(static.input_ids)).astype(np.float32)
    o.units["activation"][np.asarray(static.input_ids)] = x
    o.forward()
    util = [c[gc.UTIL.name] for c in o.conns]
    to = [c["to_id"] for c in o.conns]
    live = [c["dead"] == 0 for c in o.conns]
    w = [c["weight"] for c in o.conns]
    is_in = np.zeros(n, bool)
    is_in[np.asarray(static.input_ids)] = True
    fin = ~is_in & (o.units["level"] >= 1)
    for field, ufunc, ident, term in (
        (gc.MN, np.minimum, np.inf, lambda b: util[b]),
        (gc.PR, np.multiply, 1.0, lambda b: util[b]),
        (gc.MX, np.maximum, -np.inf, lambda b: np.abs(w[b]) * util[b]),
    ):
        # a destination's in-edges all come from lower buckets; in bucket order, slot order
        want = np.full(n, ident, np.float32)
        with np.errstate(invalid="ignore"):
            for b in range(len(o.conns)):
                ufunc.at(want, to[b][live[b]], term(b).astype(np.float32)[live[b]])
        got = o.units[field.name]
        assert _same(got[fin], want[fin]), f"{field.name}: {_diff(got[fin], want[fin])}"
    assert np.isnan(o.units[gc.MX.name][c0["to_id"][nan_slot]])
    assert o.units[gc.MN.name][30] == np.inf and o.units[gc.PR.name][30] == 1.0 and o.units[gc.MX.name][30] == -np.inf
