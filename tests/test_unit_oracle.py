"""The CPU unit-lifecycle oracle against the reference's unit goldens
(test_parity_goldens.py:1093-1152): update_unit, prune_unit and add_unit in
the step's phase order."""

from __future__ import annotations

import numpy as np
import pytest

import unit_cases as uc
from oracle import growth as og
from plastax_amd import _site


@pytest.mark.parametrize("name", uc.UNIT_CASES)
def test_unit_golden(name: str) -> None:
    doc = uc.load(name)
    assert doc["field_defaults"] == {"activation": 0.0}
    net = uc.golden_net(doc)
    static, units, conns = uc.golden_state(net, doc)
    before = {k: v.copy() for k, v in units.items()}
    dtypes = {s.name: np.dtype(s.dtype) for s in static.unit_fields}
    pruned_by_phase: list[int] = []
    added, overflow = 0, False
    if net.update_unit is not None:
        prog, names = _site.trace_update_unit(net.update_unit, dtypes, None)
        units = og.update_unit(prog, names, units, None)
    if net.prune_unit is not None:
        prog = _site.trace_prune_unit(net.prune_unit, dtypes, None)
        units, conns, doomed = og.prune_unit(prog, static, units, conns, None)
        pruned_by_phase = np.flatnonzero(doomed).tolist()
    if net.add_unit is not None:
        spawn = _site.trace_spawn(net.add_unit, dtypes, None)
        init, init_names = _site.trace_unit_init(net.add_unit, dtypes, None)
        units, added, overflow, _ = og.add_unit(spawn, init, init_names, static, net.max_levels, units, None)
    uc.check_against_golden(doc, before, units, conns, pruned_by_phase, added, overflow)


def test_every_unit_golden_is_consumed() -> None:
    assert len(uc.UNIT_CASES) == 7
