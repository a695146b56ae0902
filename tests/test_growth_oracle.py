"""The CPU growth oracle against the reference's growth goldens.

The checks mirror the reference's own golden tests
(tests/test_parity_goldens.py:478-969): the committed edge set, the grown
count and the flags, for every propose / score / claim case. The goldens are
independent of this build (emitted by the reference's scripts/parity/emit.py
from its neutral spec), so they pin the oracle's restatement and the site
program tracer together.
"""

from __future__ import annotations

import numpy as np
import pytest

import growth_cases as gc
from oracle import growth as og
from plastax_amd.growth_config import GrowthConfig


def whole_grown(doc: dict) -> int:
    return int(doc["step_growth"]["expect"]["grown"])


def _grow(hn: gc.HostNet) -> og.GrowthResult:
    return og.add_conn(
        hn.net, hn.static, hn.units, hn.conns, step=hn.step, globals_=hn.globals_,
        tail_start=hn.tail_start, units_added=hn.units_added,
    )


@pytest.mark.parametrize("name", gc.PROPOSE_CASES)
def test_propose_golden(name: str) -> None:
    doc = gc.load(name)
    hn = gc.propose_net(doc)
    res = _grow(hn)
    grown = gc.grown_pairs(hn.conns, res.conns)
    assert grown == gc.want_commits(doc["expect"]), name
    assert res.grown == doc["expect"]["grown"] == len(grown)
    assert res.needs_resort == doc["expect"]["needs_resort"]


@pytest.mark.parametrize("name", gc.SCORE_CASES)
def test_score_golden(name: str) -> None:
    """Runs A, B and C of the reference's harness (test_parity_goldens.py:795-834)."""
    doc = gc.load(name)
    free_slots = int(doc["params"]["free_slots"])
    expect = doc["expect"]
    want = gc.want_commits(expect)
    level = {u["id"]: u["level"] for u in doc["initial_units"]}

    hn = gc.score_net(doc, step_cap=None, free_at={})
    res_a = _grow(hn)
    selected = gc.grown_pairs(hn.conns, res_a.conns)
    assert not res_a.overflow
    assert res_a.grown == len(selected)
    assert (len(selected) > free_slots) == expect["conn_overflow"]

    hn = gc.score_net(doc, step_cap=free_slots, free_at={})
    res_b = _grow(hn)
    assert gc.grown_pairs(hn.conns, res_b.conns) == want
    assert res_b.grown == expect["grown"]
    assert res_b.needs_resort == expect["needs_resort"]

    per_level: dict[int, int] = {}
    for s_id, _, _ in selected:
        per_level[level[s_id]] = per_level.get(level[s_id], 0) + 1
    free_at, left = {}, free_slots
    for lvl in sorted(per_level):
        free_at[lvl] = min(left, per_level[lvl])
        left -= free_at[lvl]
    hn = gc.score_net(doc, step_cap=None, free_at=free_at)
    res_c = _grow(hn)
    assert gc.grown_pairs(hn.conns, res_c.conns) == want
    assert res_c.overflow == expect["conn_overflow"]
    assert res_c.needs_resort == expect["needs_resort"]


@pytest.mark.parametrize("name", gc.CLAIM_TOPO_CASES)
def test_claim_topological_golden(name: str) -> None:
    """The attempt with strict per-level free counts, and the whole step's
    growth over buckets that large from the start (test_parity_goldens.py:863-930)."""
    doc = gc.load(name)
    free = {int(k): v for k, v in doc["params"]["free_per_level"].items()}
    hn = gc.score_net(doc, step_cap=None, free_at=free)
    assert len(hn.static.level_capacities) == len(free)
    res = _grow(hn)
    expect = doc["expect"]
    assert gc.grown_pairs(hn.conns, res.conns) == gc.want_commits(expect)
    assert res.grown == expect["grown"]
    assert res.overflow == expect["conn_overflow"]
    assert res.needs_resort == expect["needs_resort"]
    full = [b for b, conns in enumerate(res.conns) if not conns["dead"].any()]
    assert full == expect["regrow_levels"]

    # The Driver's regrow and the same-step retry of the dropped winners.
    static, conns = hn.static, res.conns
    for lvl in full:
        static, conns = og.grow_bucket(static, conns, lvl)
    retry = doc["retry"]
    conns = gc.pin_free(conns, doc["initial_units"], {int(k): v for k, v in retry["free_per_level"].items()})
    r2 = og.retry(GrowthConfig.of(hn.net, static), hn.units, conns, res.remainder, hn.tail_start)
    assert gc.grown_pairs(conns, r2.conns) == gc.want_commits(retry["expect"])
    assert r2.overflow == retry["expect"]["conn_overflow"]
    assert not any(c["growable"].any() for c in r2.remainder[0])
    assert res.grown + r2.grown == whole_grown(doc)
    assert (res.needs_resort or r2.needs_resort) == (expect["needs_resort"] or retry["expect"]["needs_resort"])

    whole = doc["step_growth"]
    step_free = {int(k): v for k, v in whole["free_per_level"].items()}
    hn_w = gc.score_net(doc, step_cap=None, free_at=step_free)
    res_w = _grow(hn_w)
    assert gc.grown_pairs(hn_w.conns, res_w.conns) == gc.want_commits(whole["expect"])
    assert not res_w.overflow
    assert res_w.grown == whole["expect"]["grown"]


@pytest.mark.parametrize("name", gc.CLAIM_PIPE_CASES)
def test_claim_pipeline_golden(name: str) -> None:
    doc = gc.load(name)
    hn = gc.pipeline_net(doc)
    res = _grow(hn)
    expect = doc["expect"]
    assert gc.grown_pairs(hn.conns, res.conns) == gc.want_commits(expect)
    assert res.overflow == expect["conn_overflow"]
    assert res.needs_resort == expect["needs_resort"]
    assert res.tail_start - hn.tail_start == expect["tail_used"]
    assert res.conns[0]["dead"][res.tail_start:].all()


def test_every_growth_golden_is_consumed() -> None:
    used = set(gc.PROPOSE_CASES) | set(gc.SCORE_CASES) | set(gc.CLAIM_TOPO_CASES) | set(gc.CLAIM_PIPE_CASES)
    assert used == set(gc.names(lambda d: True))
    assert len(used) == 48
