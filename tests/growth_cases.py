"""The reference's growth golden cases, rebuilt on plastax_amd's API.

Each ``grow_*.json`` fixture (copied from the reference's tests/golden/,
emitted by its scripts/parity/emit.py) names registry rules and knobs; the
helpers here turn them into plastax_amd growth rules and networks exactly as
the reference's harness does (tests/test_parity_goldens.py:400-980):

- the propose rules of ``_make_propose_rule`` (:418-461): per-unit
  ``src = i``, per-connection ``src = c[FROM_ID, cid]``, global
  ``src = rng.uniform_int(n)``; ``dst = rng.uniform_int(n)``; score
  ``floor(uniform * 256) / 256``;
- the score rules of ``_make_score_rule`` (:574-668): ``grid_score_v1``,
  ``score_act_v1``, ``predicate_score_v1`` through ``predicate_add_conn``,
  ``importance_v1``, ``threshold(g)`` / ``when(g)`` from the globals;
- ``grow_init_v1``: weight ``(((3 src + 5 dst) % 16) - 8) / 8``;
- ``pin_free`` (:671-700) plugs surplus dead slots with zero-weight
  self-loops so a bucket has exactly the free slots a case pins.
"""

from __future__ import annotations

import json
import pathlib
from typing import Any

import numpy as np

import plastax_amd as px
import plastax_amd.numpy as jnp
from plastax_amd.growth_config import predicate_add_conn
from plastax_amd.state import column_to_numpy
from nets import ReluForward

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def load(name: str) -> dict[str, Any]:
    return json.loads((GOLDEN / f"{name}.json").read_text())


def names(predicate: Any) -> list[str]:
    out = []
    for path in sorted(GOLDEN.glob("grow_*.json")):
        doc = json.loads(path.read_text())
        if predicate(doc):
            out.append(path.stem)
    return out


PROPOSE_CASES = names(lambda d: "propose" in d["rules"])
SCORE_CASES = names(lambda d: "score" in d["rules"] and "model" not in d["params"])
CLAIM_TOPO_CASES = names(lambda d: d["params"].get("model") == "topological")
CLAIM_PIPE_CASES = names(lambda d: d["params"].get("model") == "pipeline")


def dyadic_weight(src: Any, dst: Any) -> Any:
    """grow_init_v1's weight: (((3*src + 5*dst) % 16) - 8) / 8."""
    return (((3 * src + 5 * dst) % 16) - 8).astype(jnp.float32) / jnp.float32(8.0)


def registry_score(rng: Any) -> Any:
    """floor(uniform * 256) / 256."""
    return jnp.floor(rng.uniform() * jnp.float32(256.0)) / jnp.float32(256.0)


def grid_score_v1(src: Any, dst: Any) -> Any:
    return (((3 * src + 5 * dst) % 17) - 8).astype(jnp.float32) / jnp.float32(8.0)


def importance_v1(i: Any) -> Any:
    return ((7 * i) % 13).astype(jnp.float32) / jnp.float32(4.0)


def propose_rule(doc: dict[str, Any], n_units: int) -> Any:
    params = doc["params"]
    kind = params["proposer"]

    class Rule(px.ProposeAddConn):
        proposer = kind
        proposals_per_proposer = int(params["proposals_per_proposer"])
        max_new_per_level = int(params["max_new_per_level"])
        max_level_gap = int(params["max_level_gap"])
        dedupe_live = bool(params.get("dedupe_live", False))
        dedupe_step = bool(params.get("dedupe_step", False))

        def propose(self, *args: Any) -> tuple[Any, Any, Any]:
            if kind == "per_unit":
                u, i, j, g, rng = args
                src = jnp.asarray(i, jnp.int32)
            elif kind == "per_connection":
                u, c, cid, j, g, rng = args
                src = jnp.asarray(c[px.FROM_ID, cid], jnp.int32)
            else:
                u, j, g, rng = args
                src = rng.uniform_int(n_units).astype(jnp.int32)
            dst = rng.uniform_int(n_units).astype(jnp.int32)
            return src, dst, registry_score(rng)

        def init(self, u: Any, src: Any, dst: Any, g: Any) -> Any:
            return px.ConnWrite.of((px.WEIGHT, dyadic_weight(src, dst)))

    return Rule()


def score_rule(doc: dict[str, Any], *, step_cap: int | None) -> Any:
    params = doc["params"]
    rules = doc["rules"]
    score_kind = rules["score"]

    def init(u: Any, src: Any, dst: Any, g: Any) -> Any:
        return px.ConnWrite.of((px.WEIGHT, dyadic_weight(src, dst)))

    knobs: dict[str, Any] = {
        "max_level_gap": int(params["max_level_gap"]),
        "selection": params["selection"],
        "direction": params.get("direction", "any"),
        "allow_self_loops": bool(params.get("allow_self_loops", False)),
        "dedupe_live": bool(params.get("dedupe_live", False)),
        "dedupe_step": bool(params.get("dedupe_step", False)),
    }
    if "max_new_per_level" in params:
        knobs["max_new_per_level"] = int(params["max_new_per_level"])
    if "level_cap_scope" in params:
        knobs["level_cap_scope"] = params["level_cap_scope"]
    caps = [c for c in (params.get("max_new_per_step"), step_cap) if c is not None]
    if caps:
        knobs["max_new_per_step"] = int(min(caps))
    trigger = doc.get("trigger")
    if trigger is not None:
        knobs["trigger"] = ("every", int(trigger["n"])) if trigger["kind"] == "every" else trigger["kind"]

    if score_kind == "predicate_score_v1":
        assert knobs.pop("selection") == "all"
        assert knobs.pop("dedupe_step") is True

        def should_add(u: Any, src: Any, dst: Any, g: Any) -> Any:
            return (src + dst) % 2 == 0

        return predicate_add_conn(should_add, init, **knobs)

    class Rule(px.ScoreAddConn):
        if params["candidates"] in ("shortlist", "shortlist_per_level"):
            candidates = params["candidates"]
            shortlist_size = int(params["shortlist_size"])

        def score(self, u: Any, src: Any, dst: Any, g: Any) -> Any:
            if score_kind == "score_act_v1":
                return u[px.ACTIVATION, src] + u[px.ACTIVATION, dst]
            return grid_score_v1(src, dst)

        def importance(self, u: Any, i: Any, g: Any) -> Any:
            return importance_v1(i)

        def threshold(self, g: Any) -> Any:
            return g["threshold"]

        def when(self, g: Any) -> Any:
            return g["when"]

        def init(self, u: Any, src: Any, dst: Any, g: Any) -> Any:
            return init(u, src, dst, g)

    for key, value in knobs.items():
        setattr(Rule, key, value)
    return Rule()


class HostNet:
    """A golden case's network as host arrays (logical arena)."""

    def __init__(self, net: Any, static: Any, units: dict, conns: list[dict], globals_: Any,
                 step: int, units_added: int = 0, tail_start: int = 0) -> None:
        self.net = net
        self.static = static
        self.units = units
        self.conns = conns
        self.globals_ = globals_
        self.step = step
        self.units_added = units_added
        self.tail_start = tail_start


def _host(state: Any, static: Any) -> tuple[dict, list[dict]]:
    uspecs = {s.name: s for s in static.unit_fields}
    cspecs = {s.name: s for s in static.conn_fields}
    units = {k: column_to_numpy(v, uspecs[k]) for k, v in state.units.items()}
    conns = [{k: column_to_numpy(v, cspecs[k]) for k, v in b.items()} for b in state.conns]
    return units, conns


def pin_free(conns: list[dict], units_doc: list[dict], free_at: dict[int, int]) -> list[dict]:
    out = [dict(b) for b in conns]
    for lvl, free in free_at.items():
        bucket = {k: v.copy() for k, v in out[lvl].items()}
        dead = np.flatnonzero(bucket["dead"])
        assert dead.size >= free, "bucket built too small to pin"
        surplus = dead[free:]
        plug = next(u["id"] for u in units_doc if u["level"] == lvl)
        bucket["dead"][surplus] = False
        bucket["from_id"][surplus] = plug
        bucket["to_id"][surplus] = plug
        bucket["weight"][surplus] = 0.0
        out[lvl] = bucket
    return out


def propose_net(doc: dict[str, Any]) -> HostNet:
    params = doc["params"]
    units = doc["initial_units"]
    n = len(units)
    rule = propose_rule(doc, n)

    class Net(px.Network):
        forward_pass = ReluForward()
        add_conn = rule
        seed = int(params["network_seed"])
        propagation = px.Propagation.TOPOLOGICAL

    edges = doc["initial_edges"]
    static, state = px.NetworkBuilder.from_edges(
        Net, n,
        np.asarray([e["src"] for e in edges], dtype=np.int32),
        np.asarray([e["dst"] for e in edges], dtype=np.int32),
        weights=np.asarray([e["fields"]["weight"] for e in edges], dtype=np.float32),
        input_ids=[u["id"] for u in units if u["is_input"]],
        output_ids=[u["id"] for u in units if u["is_output"]],
        globals_=None, capacity_headroom=4.0, device="cpu",
    )
    hu, hc = _host(state, static)
    touched = {e["src"] for e in edges} | {e["dst"] for e in edges}
    for u in units:
        if u["id"] in touched:
            assert hu["level"][u["id"]] == u["level"], f"unit {u['id']} level"
    return HostNet(Net, static, hu, hc, None, int(params["step"]))


def score_net(doc: dict[str, Any], *, step_cap: int | None, free_at: dict[int, int],
              mode: px.Propagation = px.Propagation.TOPOLOGICAL) -> HostNet:
    params = doc["params"]
    units = doc["initial_units"]
    n = len(units)
    rule = score_rule(doc, step_cap=step_cap)

    class Net(px.Network):
        forward_pass = ReluForward()
        add_conn = rule
        seed = int(params["network_seed"])
        propagation = mode

    edges = doc["initial_edges"]
    trigger = doc.get("trigger") or {}
    globals_ = {
        "threshold": np.float32(params.get("threshold", 0.0)),
        "when": np.bool_(trigger.get("value", True)),
    }
    static, state = px.NetworkBuilder.from_edges(
        Net, n,
        np.asarray([e["src"] for e in edges], dtype=np.int32),
        np.asarray([e["dst"] for e in edges], dtype=np.int32),
        weights=np.asarray([e["fields"]["weight"] for e in edges], dtype=np.float32),
        input_ids=[u["id"] for u in units if u["is_input"]],
        output_ids=[u["id"] for u in units if u["is_output"]],
        globals_=globals_, capacity_headroom=4.0, device="cpu",
    )
    hu, hc = _host(state, static)
    for u in units:
        assert hu["level"][u["id"]] == u["level"], f"unit {u['id']} level"
    if free_at:
        hc = pin_free(hc, units, free_at)
    if "batch_activations" in doc:
        per_sample = np.asarray(doc["batch_activations"], dtype=np.float32)
        hu["activation"] = (per_sample.sum(axis=0, dtype=np.float32) / np.float32(per_sample.shape[0])).astype(np.float32)
    else:
        hu["activation"] = np.asarray([u["fields"]["activation"] for u in units], dtype=np.float32)
    step = int(trigger.get("step", params["step"]))
    return HostNet(Net, static, hu, hc, globals_, step, int(trigger.get("units_added_this_step", 0)),
                   int(state.tail_start))


def pipeline_net(doc: dict[str, Any]) -> HostNet:
    """The pipeline claim case: one bucket of live edges, the golden's dead
    edges, then ``tail`` never-used slots (test_parity_goldens.py:933-966)."""
    import dataclasses

    params = doc["params"]
    hn = score_net(doc, step_cap=None, free_at={}, mode=px.Propagation.PIPELINE)
    live = len(doc["initial_edges"])
    dead_edges = doc["initial_dead_edges"]
    capacity = live + len(dead_edges) + int(params["tail"])
    bucket = {}
    for spec in hn.static.conn_fields:
        col = np.full((capacity,), spec.default, dtype=spec.dtype)
        col[:live] = hn.conns[0][spec.name][:live]
        bucket[spec.name] = col
    for i, e in enumerate(dead_edges, start=live):
        bucket["from_id"][i] = e["src"]
        bucket["to_id"][i] = e["dst"]
        bucket["dead"][i] = True
    assert hn.tail_start == live
    hn.static = dataclasses.replace(hn.static, level_capacities=(capacity,))
    hn.conns = [bucket]
    hn.tail_start = live + len(dead_edges)
    return hn


def live_pairs(conns: list[dict]) -> list[tuple[int, int, float]]:
    out = []
    for b in conns:
        dead = b["dead"].astype(bool)
        for s, d, w in zip(b["from_id"][~dead], b["to_id"][~dead], b["weight"][~dead]):
            out.append((int(s), int(d), float(w)))
    return sorted(out)


def grown_pairs(before: list[dict], after: list[dict]) -> list[tuple[int, int, float]]:
    grown = live_pairs(after)
    for pair in live_pairs(before):
        grown.remove(pair)
    return grown


def want_commits(expect: dict[str, Any]) -> list[tuple[int, int, float]]:
    return sorted(
        (int(c["src"]), int(c["dst"]), float(np.float32((((3 * c["src"] + 5 * c["dst"]) % 16) - 8) / 8.0)))
        for c in expect["committed"]
    )
