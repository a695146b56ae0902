"""The reference's unit-lifecycle goldens, rebuilt on plastax_amd's API.

Each ``unit_*.json`` fixture (copied from the reference's tests/golden/)
names registry rules; they are restated here as plastax_amd policies exactly
as the reference's harness declares them (tests/test_parity_goldens.py:
981-1032): ``unit_update_v1`` adds 1/8 to the activation,
``unit_prune_v1`` prunes below -1/2, ``unit_spawn_v1`` spawns at or above
1/2 one level deeper (``unit_spawn_deep_v1``: +30000, clamped), and
``unit_child_init_v1`` gives the child half its parent's activation. The
initial state carries the golden's own field values, levels and pruned flags
(:1053-1090).
"""

from __future__ import annotations

import json
import pathlib
from typing import Any

import numpy as np

import plastax_amd as px
import plastax_amd.numpy as jnp
from nets import ReluForward
from plastax_amd.state import column_to_numpy

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
UNIT_CASES = sorted(p.stem for p in GOLDEN.glob("unit_*.json"))


def load(name: str) -> dict[str, Any]:
    return json.loads((GOLDEN / f"{name}.json").read_text())


class UnitUpdateV1(px.UpdateUnit):
    def update(self, u, i, g):
        return px.UnitWrite.of((px.ACTIVATION, u[px.ACTIVATION, i] + 0.125))


class UnitPruneV1(px.PruneUnit):
    def predicate(self, u, i, g):
        return u[px.ACTIVATION, i] < jnp.float32(-0.5)


class UnitSpawnV1(px.AddUnit):
    offset = 1

    def spawn(self, u, parent, g):
        return u[px.ACTIVATION, parent] >= jnp.float32(0.5), jnp.int32(self.offset)

    def init(self, u, child, parent, g):
        return px.UnitWrite.of((px.ACTIVATION, u[px.ACTIVATION, parent] / 2))


class UnitSpawnDeepV1(UnitSpawnV1):
    offset = 30000


RULES = {
    "unit_update_v1": UnitUpdateV1,
    "unit_prune_v1": UnitPruneV1,
    "unit_spawn_v1": UnitSpawnV1,
    "unit_spawn_deep_v1": UnitSpawnDeepV1,
}


def golden_net(doc: dict[str, Any]) -> type:
    rules = doc["rules"]

    def rule(slot: str) -> Any:
        return RULES[rules[slot]]() if slot in rules else None

    class Net(px.Network):
        forward_pass = ReluForward()
        update_unit = rule("update_unit")
        prune_unit = rule("prune_unit")
        add_unit = rule("add_unit")
        unit_capacity = int(doc["capacity"])
        max_levels = int(doc["max_levels"])
        propagation = px.Propagation.TOPOLOGICAL

    return Net


def golden_state(net: type, doc: dict[str, Any]) -> tuple[Any, dict, list[dict]]:
    """(static, host units, host conns) of the golden's initial network."""
    units = doc["initial_units"]
    edges = doc["initial_edges"]
    static, state = px.NetworkBuilder.from_edges(
        net, len(units),
        np.asarray([e["src"] for e in edges], dtype=np.int32),
        np.asarray([e["dst"] for e in edges], dtype=np.int32),
        weights=np.asarray([e["fields"]["weight"] for e in edges], dtype=np.float32),
        input_ids=[u["id"] for u in units if u["is_input"]],
        output_ids=[u["id"] for u in units if u["is_output"]],
        globals_=None, device="cpu")
    assert static.num_units == doc["capacity"]
    uspecs = {s.name: s for s in static.unit_fields}
    cspecs = {s.name: s for s in static.conn_fields}
    hu = {k: column_to_numpy(v, uspecs[k]).copy() for k, v in state.units.items()}
    hc = [{k: column_to_numpy(v, cspecs[k]).copy() for k, v in b.items()} for b in state.conns]
    ids = np.asarray([u["id"] for u in units])
    hu["activation"][ids] = np.asarray([u["fields"]["activation"] for u in units], np.float32)
    hu["pruned"][ids] = np.asarray([u["pruned"] for u in units], bool)
    hu["level"][ids] = np.asarray([u["level"] for u in units], np.int32)
    return static, hu, hc


def check_against_golden(doc: dict[str, Any], before: dict, units: dict, conns: list[dict],
                         pruned_by_phase: list[int], units_added: int, overflow: bool) -> None:
    """The reference harness's assertions (test_parity_goldens.py:1127-1152)."""
    expect = doc["expect"]
    for want in expect["units"]:
        uid = want["id"]
        assert units["activation"][uid] == want["fields"]["activation"], f"unit {uid} activation"
        assert bool(units["pruned"][uid]) == want["pruned"], f"unit {uid} pruned"
        assert units["level"][uid] == want["level"], f"unit {uid} level"
    assert pruned_by_phase == expect["pruned"]
    assert units_added == len(expect.get("children", []))
    assert overflow == expect.get("unit_overflow", False)
    n = len(expect["units"])
    assert units["pruned"][n:].all()
    for col, old in before.items():
        np.testing.assert_array_equal(units[col][n:], old[n:], err_msg=col)
    live = []
    for b in conns:
        d = b["dead"].astype(bool)
        live += [(int(s), int(t), float(w)) for s, t, w in zip(b["from_id"][~d], b["to_id"][~d], b["weight"][~d])]
    want_edges = sorted((int(e["src"]), int(e["dst"]), float(e["fields"]["weight"])) for e in expect["edges"])
    assert sorted(live) == want_edges
