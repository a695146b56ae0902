"""The growth API names of the reference's public surface: ``px.Proposal``
(traits.py:554-566), ``shortlist_coverage`` / ``recommended_shortlist`` /
``ShortlistCoverage`` (phases.py:3560-3650), and the constant tables a
proposer like examples/dst_sparse.py:318-330 indexes with traced integers.

The traced table reads are checked against an eager restatement of jnp's
gather semantics (a negative index counts from the end, then the index is
clamped), evaluated by the oracle's site interpreter at every index in and
around the table."""

from __future__ import annotations

import numpy as np
import pytest

import plastax_amd as px
import plastax_amd.numpy as jnp
from plastax_amd import _site


def test_proposal_is_a_namedtuple_of_src_dst_score() -> None:
    p = px.Proposal(src=1, dst=2, score=0.5)
    assert p._fields == ("src", "dst", "score")
    assert tuple(p) == (1, 2, 0.5)
    assert p.src == 1 and p.dst == 2 and p.score == 0.5


class _Tables:
    """A score that reads constant tables at traced indices, as the RigL
    proposer of examples/dst_sparse.py reads its layer tables."""

    def __init__(self) -> None:
        sizes = np.asarray([5, 7, 3, 4], np.int32)
        starts = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
        self.next_start = jnp.asarray(starts[1:])
        self.next_width = jnp.asarray(np.append(sizes[1:], 0).astype(np.int32))
        self.gain = jnp.asarray(np.float32([0.5, -1.25, 3.0, 0.0625]))

    def score(self, u, src, dst, g):
        layer = jnp.sum(src >= self.next_start)  # booleans counted as int32
        width = self.next_width[layer]
        far = self.gain[dst - 9]  # negative and past-the-end indices
        return width.astype(jnp.float32) * jnp.float32(10.0) + far + layer.astype(jnp.float32) * jnp.float32(100.0)


def _jnp_take(table: np.ndarray, k: np.ndarray) -> np.ndarray:
    k = np.where(k < 0, k + table.size, k)
    return table[np.clip(k, 0, table.size - 1)]


def test_constant_tables_follow_jnp_gather_semantics(oracle) -> None:
    from oracle import growth as og

    rule = _Tables()
    prog = _site.trace_score(rule, {"level": np.dtype(np.int32)}, None)
    src, dst = np.meshgrid(np.arange(-3, 24, dtype=np.int32), np.arange(-2, 20, dtype=np.int32))
    src, dst = src.ravel(), dst.ravel()
    units = {"level": np.zeros(24, np.int32)}
    (got,) = og.site_eval(prog, src.size, {"src": src, "dst": dst}, units, None)
    starts = np.asarray(rule.next_start).view(np.ndarray)
    layer = np.sum(src[:, None] >= starts[None, :], axis=1).astype(np.int32)
    width = _jnp_take(np.asarray(rule.next_width).view(np.ndarray), layer)
    far = _jnp_take(np.asarray(rule.gain).view(np.ndarray), dst - 9)
    want = (width.astype(np.float32) * np.float32(10.0) + far + layer.astype(np.float32) * np.float32(100.0))
    assert np.array_equal(np.asarray(got, np.float32).view(np.uint32), want.astype(np.float32).view(np.uint32))
    # eager reads of a table stay plain numpy reads
    assert int(rule.next_width[1]) == 3 and rule.next_start[1:].tolist() == [12, 15, 19]


def test_traced_index_must_be_an_integer() -> None:
    table = jnp.asarray(np.float32([1.0, 2.0]))

    class Bad:
        def score(self, u, src, dst, g):
            return table[src.astype(jnp.float32)]

    with pytest.raises(px.UnsupportedPolicyError):
        _site.trace_score(Bad(), {}, None)


def _layered_state(layers, gap):
    rng = np.random.default_rng(0)
    base = np.concatenate([[0], np.cumsum(layers)])
    src, dst = [], []
    for l in range(len(layers) - 1):
        for j in range(base[l + 1], base[l + 2]):
            src.append(int(rng.integers(base[l], base[l + 1])))
            dst.append(j)
    src = np.asarray(src, np.int32)
    dst = np.asarray(dst, np.int32)

    class Grow(px.ScoreAddConn):
        candidates = "shortlist_per_level"
        shortlist_size = 8
        max_new_per_level = 4
        max_level_gap = gap

        def score(self, u, s, d, g):
            return jnp.float32(0.0)

        def importance(self, u, i, g):
            return jnp.float32(1.0)

        def init(self, u, s, d, g):
            return px.ConnWrite.of((px.WEIGHT, jnp.float32(0.0)))

    class Net(px.Network):
        add_conn = Grow()

    static, state = px.NetworkBuilder.from_edges(
        Net, int(base[-1]), src, dst, weights=np.zeros(src.size, np.float32),
        input_ids=np.arange(layers[0]), output_ids=np.arange(base[-2], base[-1]), globals_=None)
    return Net, static, state


@pytest.mark.parametrize("gap", [1, 2])
def test_shortlist_coverage_counts_each_buckets_window(gap: int) -> None:
    layers = [6, 16, 8, 4]
    net, static, state = _layered_state(layers, gap)
    cov = px.shortlist_coverage(net, static, state)
    # a growing net gives its deepest level a bucket too (nothing deeper: no destination)
    assert len(cov) == len(static.level_capacities) == 4
    for b, c in enumerate(cov):
        assert isinstance(c, px.ShortlistCoverage)
        dests = sum(layers[b + 1: b + 1 + gap])
        assert (c.bucket, c.candidate_units, c.source_units, c.destination_units) == (b, 8, layers[b], dests)
        assert c.covered == (8 >= dests)
    assert px.recommended_shortlist(net, static, state) == max(sum(layers[b + 1: b + 1 + gap]) for b in range(4))


def test_no_shortlist_reports_nothing() -> None:
    net, static, state = _layered_state([6, 16, 8, 4], 1)

    class Exhaustive(net):
        pass

    Exhaustive.add_conn = type("G", (), {"candidates": "exhaustive"})()
    assert px.shortlist_coverage(Exhaustive, static, state) == ()
    assert px.recommended_shortlist(Exhaustive, static, state) == 0
