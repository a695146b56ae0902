"""Pins of the oracle's primitives that do not depend on the device.

- Philox-4x32-10 against the Random123 known-answer vectors (Salmon et al.,
  SC'11; the plastax mapping of rng.py:109-141 makes the all-zero and
  all-ones blocks diagonal, so those two KATs apply to philox32 directly).
- exp / log / tanh / sigmoid within 2 ulp of the double-precision functions
  over the float32 range, and their special values.
- The Adam power b^t (integer t) equal to the correctly rounded power, from
  exact rational arithmetic.
"""

from __future__ import annotations

import ctypes
import math
from fractions import Fraction

import numpy as np
import pytest

import plastax_amd as px

KATS = [
    # (ctr[4], key[2]) -> out[4]   (Random123 kat_vectors, philox4x32_10)
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    (
        (0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344),
        (0xA4093822, 0x299F31D0),
        (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1),
    ),
]


@pytest.mark.parametrize("ctr,key,want", KATS)
def test_philox_core_matches_random123_kats(oracle, ctr, key, want) -> None:
    lib = oracle.load()
    c = (ctypes.c_uint32 * 4)(*ctr)
    k = (ctypes.c_uint32 * 2)(*key)
    out = (ctypes.c_uint32 * 4)()
    lib.ox_philox4x32_10(c, k, out)
    assert tuple(out) == want


def test_plastax_philox_mapping_on_diagonal_kats(oracle) -> None:
    lib = oracle.load()
    assert lib.ox_philox32(0, 0) == 0x6627E8D5
    assert lib.ox_philox32(2**64 - 1, 2**64 - 1) == 0x408F276D
    assert int(px.rng.philox32(0, 0)) == 0x6627E8D5
    assert int(px.rng.philox32(np.uint64(2**64 - 1), np.uint64(2**64 - 1))) == 0x408F276D


def test_host_rng_matches_oracle_words(oracle) -> None:
    lib = oracle.load()
    rng = np.random.default_rng(0)
    seeds = rng.integers(0, 2**63, 500, dtype=np.int64).astype(np.uint64)
    ctrs = rng.integers(0, 2**63, 500, dtype=np.int64).astype(np.uint64)
    words = px.rng.philox32(seeds, ctrs)
    assert [int(w) for w in words] == [lib.ox_philox32(int(s), int(c)) for s, c in zip(seeds, ctrs)]
    # site contract (rng.py:10-56): draw = philox(site_seed, (j<<16)|sub)
    site = px.rng.site_seed(7, np.uint32(3), 1, np.uint64(42))
    assert int(site) == lib.ox_site_seed(7, 3, 1, 42)
    assert int(px.rng.draw(site, np.uint64(5), 2)) == lib.ox_site_draw(int(site), 5, 2)
    w = px.rng.philox32(seeds[:50], ctrs[:50])
    for n in (1, 2, 3, 10, 1000):
        got = px.rng.uniform_int(w, n)
        assert [int(v) for v in got] == [lib.ox_uniform_int(int(x), n) for x in w]
        assert int(got.max()) < n


def _ulps(got: float, exact: float) -> float:
    if math.isnan(exact):
        return 0.0 if math.isnan(got) else math.inf
    if math.isinf(exact):
        return 0.0 if got == exact else math.inf
    spacing = float(np.spacing(np.float32(abs(exact))))
    return abs(got - exact) / spacing


@pytest.mark.parametrize(
    "name,ref,lo,hi",
    [
        ("ox_expf", math.exp, -87.0, 88.5),
        ("ox_tanhf", math.tanh, -12.0, 12.0),
        ("ox_sigmoidf", lambda x: 1.0 / (1.0 + math.exp(-x)), -30.0, 30.0),
    ],
)
def test_elementary_functions_within_two_ulp(oracle, name, ref, lo, hi) -> None:
    fn = getattr(oracle.load(), name)
    rng = np.random.default_rng(1)
    xs = np.concatenate([rng.uniform(lo, hi, 20000), rng.uniform(-1, 1, 20000)]).astype(np.float32)
    worst = max(_ulps(fn(float(x)), ref(float(x))) for x in xs)
    assert worst <= 2.0, worst


@pytest.mark.parametrize("name,ref", [("ox_cosf", math.cos), ("ox_sinf", math.sin)])
def test_cos_sin_accuracy(oracle, name, ref) -> None:
    """Cephes' float32 sin / cos: within 2 ulp of the exact function on
    |x| <= 64 (Box-Muller's argument is in [0, 2 pi)), and within 1e-7
    absolute up to the reduction's limit 8192, where a result near a zero of
    the function has few significant bits left (Cephes' PLOSS range)."""
    fn = getattr(oracle.load(), name)
    rng = np.random.default_rng(3)
    near = np.concatenate([rng.uniform(-64, 64, 20000), rng.uniform(0, 2 * math.pi, 20000),
                           np.float32([0.0, -0.0, 1e-38, math.pi, math.pi / 2, math.pi / 4, 2 * math.pi])])
    near = near.astype(np.float32)
    worst = max(_ulps(fn(float(x)), ref(float(x))) for x in near)
    assert worst <= 2.0, worst
    far = rng.uniform(-8192, 8192, 20000).astype(np.float32)
    assert max(abs(fn(float(x)) - ref(float(x))) for x in far) <= 1e-7


def test_log_within_two_ulp(oracle) -> None:
    fn = oracle.load().ox_logf
    rng = np.random.default_rng(2)
    xs = np.concatenate(
        [np.exp(rng.uniform(-87, 88, 20000)), rng.uniform(0.5, 2.0, 20000), [1e-40, 3e-45]]
    ).astype(np.float32)
    worst = max(_ulps(fn(float(x)), math.log(float(x))) for x in xs)
    assert worst <= 2.0, worst


@pytest.mark.parametrize("name,ref", [("ox_log1pf", math.log1p), ("ox_expm1f", math.expm1)])
def test_log1p_expm1_within_three_ulp(oracle, name, ref) -> None:
    """Kahan's log1p / expm1 over the Cephes log / exp: the cancellation of
    1 + x is exact, so the error is that of log or exp plus a few roundings
    (Goldberg's Theorem 4 bounds it by 5 eps for a correctly rounded log);
    measured here against the exact functions, including tiny |x| where the
    naive log(1 + x) / exp(x) - 1 lose every digit."""
    fn = getattr(oracle.load(), name)
    rng = np.random.default_rng(4)
    tiny = rng.uniform(-1, 1, 20000) * np.exp(rng.uniform(-80, 0, 20000))
    if name == "ox_log1pf":
        xs = np.concatenate([tiny, rng.uniform(-0.999, 10, 20000), np.exp(rng.uniform(-5, 80, 20000))])
    else:
        xs = np.concatenate([tiny, rng.uniform(-20, 20, 20000), rng.uniform(-100, 88, 20000)])
    xs = xs.astype(np.float32)
    worst = max(_ulps(fn(float(x)), ref(float(x))) for x in xs)
    assert worst <= 3.0, worst  # measured: 1.95 (log1p), 2.36 (expm1)
    # the naive formula fails where these succeed
    assert fn(1e-10) == pytest.approx(1e-10, rel=1e-6)


def test_log1p_expm1_special_values(oracle) -> None:
    lib = oracle.load()
    for fn in (lib.ox_log1pf, lib.ox_expm1f):
        assert fn(0.0) == 0.0 and math.copysign(1, fn(-0.0)) < 0
        assert fn(math.inf) == math.inf and math.isnan(fn(math.nan))
        assert fn(1e-30) == np.float32(1e-30)
    assert lib.ox_log1pf(-1.0) == -math.inf
    assert math.isnan(lib.ox_log1pf(-2.0)) and math.isnan(lib.ox_log1pf(-math.inf))
    assert lib.ox_expm1f(-math.inf) == -1.0 and lib.ox_expm1f(-200.0) == -1.0
    assert lib.ox_expm1f(100.0) == math.inf


def test_special_values(oracle) -> None:
    lib = oracle.load()
    assert lib.ox_expf(0.0) == 1.0
    assert lib.ox_expf(-200.0) == 0.0
    assert lib.ox_expf(100.0) == math.inf
    assert lib.ox_expf(-math.inf) == 0.0
    assert math.isnan(lib.ox_expf(math.nan))
    assert lib.ox_logf(1.0) == 0.0
    assert lib.ox_logf(0.0) == -math.inf
    assert math.isnan(lib.ox_logf(-1.0))
    assert lib.ox_logf(math.inf) == math.inf
    assert lib.ox_tanhf(0.0) == 0.0 and math.copysign(1, lib.ox_tanhf(-0.0)) < 0
    assert lib.ox_tanhf(50.0) == 1.0 and lib.ox_tanhf(-50.0) == -1.0
    assert lib.ox_tanhf(math.inf) == 1.0
    assert lib.ox_sigmoidf(0.0) == 0.5
    assert lib.ox_cosf(0.0) == 1.0 and lib.ox_cosf(-0.0) == 1.0
    assert lib.ox_sinf(0.0) == 0.0 and math.copysign(1, lib.ox_sinf(-0.0)) < 0
    for fn in (lib.ox_cosf, lib.ox_sinf):
        assert math.isnan(fn(math.inf)) and math.isnan(fn(-math.inf)) and math.isnan(fn(math.nan))
        assert fn(3e7) == 0.0  # past 2^24 - 1: no significant bits left


def test_adam_power_is_the_correctly_rounded_power(oracle) -> None:
    lib = oracle.load()
    for b in (np.float32(0.9), np.float32(0.999)):
        fb = Fraction(float(b))
        for t in list(range(0, 300)) + [1000, 4096, 65535, 100000]:
            exact = fb**t
            want = np.float32(float(exact))  # float() rounds the rational correctly
            got = np.float32(lib.ox_pow_step(float(b), float(t)))
            assert got == want, (float(b), t)


def test_capacity_policy_matches_reference_rules() -> None:
    """topo.py:455-506: next power of two (min 64), or a multiple of align."""
    cp = px.topo.capacity_policy
    assert cp(0) == 64 and cp(1) == 64 and cp(64) == 64 and cp(65) == 128
    assert cp(1000) == 1024 and cp(1024) == 1024 and cp(1025) == 2048
    assert cp(100, headroom=1.0) == 256
    assert cp(1000, align=256) == 1024 and cp(1, align=256) == 256 and cp(513, align=256) == 768
    with pytest.raises(ValueError):
        cp(10, headroom=-1.0)


def test_initial_levels_longest_path() -> None:
    edges = np.asarray([[0, 2], [1, 2], [2, 3], [0, 3], [3, 4], [1, 4]])
    lv = px.topo.initial_levels(5, edges)
    assert lv.tolist() == [0, 0, 1, 2, 3]
    with pytest.raises(ValueError):
        px.topo.initial_levels(3, np.asarray([[0, 1], [1, 2], [2, 0]]))
    # inputs stay at level 0 even with an edge into them
    lv = px.topo.initial_levels(3, np.asarray([[1, 0], [0, 2]]), input_ids=(0,))
    assert lv[0] == 0 and lv[2] == 1


def _levels_by_definition(n: int, edges: np.ndarray, inputs: tuple[int, ...]) -> tuple[np.ndarray, bool]:
    """Brute force on a tiny graph: the transitive closure by repeated
    squaring; a unit on a cycle reaches itself; tainted = on a cycle or
    reachable from one; an untainted unit's level is its longest incoming
    path (recursion over predecessors); a tainted one's is one more than its
    highest untainted predecessor (0 without one). Edges into inputs are
    dropped for the levels, kept for the cycle flag."""
    def closure(es):
        r = np.zeros((n, n), dtype=bool)
        for a, b in es:
            r[a, b] = True
        for _ in range(n.bit_length() + 1):
            r = r | ((r.astype(np.int64) @ r.astype(np.int64)) > 0)
        return r

    any_cycle = bool(np.diag(closure(edges)).any()) if len(edges) else False
    es = [(a, b) for a, b in edges.tolist() if b not in inputs]
    r = closure(es)
    cyc = np.diag(r).copy()
    tainted = cyc | (r[cyc].any(axis=0) if cyc.any() else np.zeros(n, bool))
    preds = {v: [a for a, b in es if b == v] for v in range(n)}
    memo: dict[int, int] = {}

    def longest(v):
        if v not in memo:
            memo[v] = max((longest(p) + 1 for p in preds[v]), default=0)
        return memo[v]

    lv = np.zeros(n, dtype=np.int32)
    for v in range(n):
        if not tainted[v]:
            lv[v] = longest(v)
        else:
            lv[v] = max((longest(p) + 1 for p in preds[v] if not tainted[p]), default=0)
    return lv, any_cycle


def test_initial_levels_match_the_definition_on_random_graphs() -> None:
    rng = np.random.default_rng(3)
    for _ in range(400):
        n = int(rng.integers(1, 12))
        m = int(rng.integers(0, 25))
        edges = np.stack([rng.integers(0, n, m), rng.integers(0, n, m)], 1)
        if rng.random() < 0.5:
            edges = edges[edges[:, 0] < edges[:, 1]]
        inputs = tuple(sorted(set(rng.integers(0, n, int(rng.integers(0, 3))).tolist())))
        want, cyclic = _levels_by_definition(n, edges, inputs)
        got = px.topo.initial_levels(n, edges, allow_cycles=True, input_ids=inputs)
        assert got.tolist() == want.tolist(), (n, edges.tolist(), inputs)
        if cyclic:
            with pytest.raises(ValueError, match="cycle"):
                px.topo.initial_levels(n, edges, input_ids=inputs)
        else:
            assert px.topo.initial_levels(n, edges, input_ids=inputs).tolist() == want.tolist()


def test_initial_levels_of_a_chain_deeper_than_the_quick_rounds() -> None:
    n = 200
    chain = np.stack([np.arange(n - 1), np.arange(1, n)], 1)
    assert px.topo.initial_levels(n, chain).tolist() == list(range(n))
    ring = np.concatenate([chain, [[n - 1, 150]]])
    with pytest.raises(ValueError, match="cycle"):
        px.topo.initial_levels(n, ring)
    lv = px.topo.initial_levels(n, ring, allow_cycles=True)
    # 150 enters the cycle from 149; the rest of the cycle has no untainted predecessor
    assert lv[:151].tolist() == list(range(151)) and not lv[151:].any()
