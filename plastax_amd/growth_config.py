"""Growth-rule knobs, read and validated once when a step is built.

The reference reads a growth rule's attributes structurally
(phases.py:4628-4698) after ``_validate_growth_knobs`` (traits.py:1390-1515)
has checked them; ``GrowthConfig.of`` does both for the device path and
computes the static sizes the phase needs (candidate pool, per-level budget
``k``). ``predicate_add_conn`` is the reference's boolean adapter
(traits.py:1517-1562).
"""

from __future__ import annotations

import dataclasses
from typing import Any, Callable, NamedTuple

import numpy as np

from plastax_amd._types import Propagation

SELECTIONS = ("top_k", "threshold", "all")
LEVEL_CAP_SCOPES = ("source_level", "step")
DIRECTIONS = ("any", "deeper", "same_or_deeper")
PROPOSERS = ("per_unit", "per_connection", "global")
CANDIDATES = ("exhaustive", "shortlist", "shortlist_per_level")
ON_OVERFLOW = ("flag", "error")


def is_propose_rule(ac: Any) -> bool:
    """A ProposeAddConn (structural: it has ``propose``), else a ScoreAddConn."""
    return callable(getattr(ac, "propose", None))


@dataclasses.dataclass(frozen=True)
class GrowthConfig:
    """The static configuration of one net's add_conn phase."""

    propose: bool
    proposer: str  # per_unit / per_connection / global ("" for score rules)
    proposals: int  # P
    candidates: str  # exhaustive / shortlist / shortlist_per_level ("" for propose)
    shortlist: bool
    per_level: bool
    pool_side: int  # M (or num_units for the exhaustive grid)
    pool: int  # candidates per list (static)
    k: int  # per-level (or per-step) budget
    selection: str
    step_scope: bool
    max_new_per_step: int | None
    max_level_gap: int
    direction: str
    allow_self_loops: bool
    dedupe_live: bool
    dedupe_step: bool
    trigger: Any
    on_overflow: str
    pipeline: bool
    num_units: int
    num_buckets: int

    @staticmethod
    def of(net: Any, static: Any) -> "GrowthConfig":
        ac = net.add_conn
        name = getattr(net, "__name__", type(net).__name__)
        for removed in ("dedupe", "max_candidates", "max_candidate_units", "shortlist_per_level"):
            if hasattr(ac, removed):
                raise TypeError(f"{name}.add_conn.{removed} was removed")
        selection = str(getattr(ac, "selection", "top_k"))
        if selection not in SELECTIONS:
            raise TypeError(f"{name}.add_conn.selection must be one of {SELECTIONS}; got {selection!r}")
        mnpl = getattr(ac, "max_new_per_level", None)
        if selection != "all" or mnpl is not None:
            if not isinstance(mnpl, (int, np.integer)) or isinstance(mnpl, bool) or mnpl < 1:
                raise TypeError(
                    f"{name}.add_conn.max_new_per_level must be an int >= 1 "
                    f'(required unless selection = "all"); got {mnpl!r}'
                )
        if selection == "threshold" and not callable(getattr(ac, "threshold", None)):
            raise TypeError(f'{name}.add_conn: selection = "threshold" requires a threshold(g) method')
        scope = str(getattr(ac, "level_cap_scope", "source_level"))
        if scope not in LEVEL_CAP_SCOPES:
            raise TypeError(f"{name}.add_conn.level_cap_scope must be one of {LEVEL_CAP_SCOPES}")
        mnps = getattr(ac, "max_new_per_step", None)
        if mnps is not None and (not isinstance(mnps, (int, np.integer)) or isinstance(mnps, bool) or mnps < 1):
            raise TypeError(f"{name}.add_conn.max_new_per_step must be an int >= 1 or None")
        direction = str(getattr(ac, "direction", "any"))
        if direction not in DIRECTIONS:
            raise TypeError(f"{name}.add_conn.direction must be one of {DIRECTIONS}")
        gap = getattr(ac, "max_level_gap", 1)
        if not isinstance(gap, (int, np.integer)) or isinstance(gap, bool) or gap < 0:
            raise TypeError(f"{name}.add_conn.max_level_gap must be an int >= 0")
        trigger = getattr(ac, "trigger", "every_step")
        if isinstance(trigger, tuple):
            if len(trigger) != 2 or trigger[0] != "every" or int(trigger[1]) < 1:
                raise TypeError(f'{name}.add_conn.trigger tuple must be ("every", n >= 1)')
        elif trigger not in ("every_step", "on_units_added", "when"):
            raise TypeError(f"{name}.add_conn.trigger {trigger!r} is not a trigger")
        if trigger == "when" and not callable(getattr(ac, "when", None)):
            raise TypeError(f'{name}.add_conn: trigger = "when" requires a when(g) method')
        on_overflow = str(getattr(ac, "on_overflow", "flag"))
        if on_overflow not in ON_OVERFLOW:
            raise TypeError(f"{name}.add_conn.on_overflow must be one of {ON_OVERFLOW}")

        n = int(static.num_units)
        pipeline = static.propagation is Propagation.PIPELINE
        propose = is_propose_rule(ac)
        proposer, num_p, cand = "", 0, ""
        shortlist = per_level = False
        pool_side = n
        if propose:
            proposer = str(getattr(ac, "proposer", "per_unit"))
            if proposer not in PROPOSERS:
                raise TypeError(f"{name}.add_conn.proposer must be one of {PROPOSERS}")
            num_p = int(getattr(ac, "proposals_per_proposer", 0))
            if num_p < 1:
                raise TypeError(f"{name}.add_conn.proposals_per_proposer must be an int >= 1")
            total_slots = int(sum(static.level_capacities))
            pool = {"per_unit": n * num_p, "per_connection": total_slots * num_p, "global": num_p}[proposer]
        else:
            cand = str(getattr(ac, "candidates", "exhaustive"))
            if cand not in CANDIDATES:
                raise TypeError(f"{name}.add_conn.candidates must be one of {CANDIDATES}")
            size = getattr(ac, "shortlist_size", None)
            shortlist = cand in ("shortlist", "shortlist_per_level") and size is not None and 0 < int(size) < n
            per_level = shortlist and cand == "shortlist_per_level"
            if cand == "shortlist_per_level" and pipeline:
                raise ValueError(
                    'candidates = "shortlist_per_level" is levels-based and so '
                    "topological-only; PIPELINE networks use the global shortlist."
                )
            if shortlist and not callable(getattr(ac, "importance", None)):
                raise TypeError(f"{name}.add_conn: a shortlist requires an importance(u, i, g) method")
            pool_side = int(size) if shortlist else n
            pool = pool_side * pool_side
        k = pool if selection == "all" else max(0, min(int(mnpl), pool))
        return GrowthConfig(
            propose=propose,
            proposer=proposer,
            proposals=num_p,
            candidates=cand,
            shortlist=shortlist,
            per_level=per_level,
            pool_side=pool_side,
            pool=pool,
            k=k,
            selection=selection,
            step_scope=scope == "step" and selection != "all",
            max_new_per_step=None if mnps is None else int(mnps),
            max_level_gap=int(gap),
            direction=direction,
            allow_self_loops=bool(getattr(ac, "allow_self_loops", False)),
            dedupe_live=bool(getattr(ac, "dedupe_live", False)),
            dedupe_step=bool(getattr(ac, "dedupe_step", False)),
            trigger=trigger,
            on_overflow=on_overflow,
            pipeline=pipeline,
            num_units=n,
            num_buckets=len(static.level_capacities),
        )

    def fires(self, ac: Any, *, step: int, interval: int, units_added: int, globals_: Any) -> bool:
        """Whether the phase runs this step (phases.py:5152-5187)."""
        fire = True
        if interval > 1:
            fire = fire and step % interval == 0
        if self.trigger == "on_units_added":
            fire = fire and units_added > 0
        elif self.trigger == "when":
            fire = fire and bool(np.asarray(ac.when(globals_)))
        elif isinstance(self.trigger, tuple):
            fire = fire and step % int(self.trigger[1]) == 0
        return fire


def predicate_add_conn(should_add: Callable[..., Any], init: Callable[..., Any], **params: Any) -> Any:
    """A boolean growth predicate as a ScoreAddConn (traits.py:1517-1562):
    score 0.0 (grow) or -inf (veto), ``selection = "all"``,
    ``dedupe_step = True``; ``params`` override any knob."""
    from plastax_amd import numpy as jnp

    class PredicateAddConn:
        selection = "all"
        dedupe_step = True

        def score(self, u: Any, src: Any, dst: Any, g: Any) -> Any:
            return jnp.where(should_add(u, src, dst, g), np.float32(0.0), np.float32(-np.inf))

        def init(self, u: Any, src: Any, dst: Any, g: Any) -> Any:
            return init(u, src, dst, g)

    for key, value in params.items():
        setattr(PredicateAddConn, key, value)
    return PredicateAddConn()


class ShortlistCoverage(NamedTuple):
    """Whether one bucket's growth shortlist reaches every eligible
    destination (phases.py:3560-3575).

    bucket: the bucket (its source level); candidate_units: the shortlist
    size M; source_units / destination_units: the units at the bucket's level
    / in its growth window (deeper, within ``max_level_gap``); covered:
    M >= destination_units.
    """

    bucket: int
    candidate_units: int
    source_units: int
    destination_units: int
    covered: bool


def shortlist_coverage(net: Any, static: Any, state: Any) -> tuple[ShortlistCoverage, ...]:
    """Per bucket, whether a shortlisted ``add_conn`` can reach every
    eligible destination (phases.py:3578-3628).

    A shortlist draws candidates from the M most important sources of a
    bucket's level crossed with the M most important eligible destinations,
    so at most M distinct units of a wider destination window can ever gain
    an edge. The check reads the state's LEVEL column on the host (levels are
    runtime data). Empty when the net declares no shortlist."""
    from plastax_amd._types import LEVEL

    ac = getattr(net, "add_conn", None)
    if ac is None:
        return ()
    kind = str(getattr(ac, "candidates", "exhaustive"))
    m = getattr(ac, "shortlist_size", None) if kind != "exhaustive" else None
    if m is None:
        return ()
    col = state.units[LEVEL.name]
    levels = np.asarray(col.cpu().numpy() if hasattr(col, "cpu") else col)
    gap = int(getattr(ac, "max_level_gap", 1))
    out = []
    for b in range(len(static.level_capacities)):
        dests = int(np.count_nonzero((levels > b) & (levels <= b + gap)))
        out.append(ShortlistCoverage(bucket=b, candidate_units=int(m),
                                     source_units=int(np.count_nonzero(levels == b)),
                                     destination_units=dests, covered=int(m) >= dests))
    return tuple(out)


def recommended_shortlist(net: Any, static: Any, state: Any) -> int:
    """The smallest shortlist size that reaches every eligible destination
    of every bucket (phases.py:3631-3650): the largest destination window,
    or 0 without a shortlist. A floor only: the candidate volume rule (M
    above sqrt(churn * E)) still applies."""
    return max((c.destination_units for c in shortlist_coverage(net, static, state)), default=0)
