"""Host-side topology helpers: initial levels and bucket capacities.

``initial_levels`` computes the levels defined by src/plastax/topo.py:35-130
(a unit's level is the length of the longest edge path that ends at it,
inputs pinned to level 0); ``capacity_policy`` is topo.py:455-506.
"""

from __future__ import annotations

import math

import numpy as np

# Relaxation rounds tried before the graph is checked for cycles: enough for
# every layered net of the configurations (depth <= 9), few enough that a
# recurrent (PIPELINE) net reaches the cycle analysis quickly.
_QUICK_ROUNDS = 64


def initial_levels(
    num_units: int,
    edges: np.ndarray,
    *,
    allow_cycles: bool = False,
    input_ids: tuple[int, ...] = (),
) -> np.ndarray:
    """Level of every unit: 0 without incoming edges, else the length of the
    longest edge path that ends at the unit (topo.py:35-130).

    Edges into an input count for the cycle check but do not raise its level.
    On a cycle this raises ValueError unless ``allow_cycles``. Then a unit on
    a cycle, or reachable from one, gets one more than the highest level among
    its predecessors that are neither (0 if it has none), which is the level
    the reference's frontier walk leaves such a unit with.
    """
    e = np.asarray(edges, dtype=np.int64).reshape(-1, 2)
    src, dst = e[:, 0], e[:, 1]
    if src.size and len(input_ids):
        pinned = np.zeros(num_units, dtype=bool)
        pinned[np.asarray(input_ids, dtype=np.int64)] = True
        into_input = pinned[dst]
        if into_input.any():
            if not allow_cycles:
                _levels(num_units, src, dst, allow_cycles=False)
            src, dst = src[~into_input], dst[~into_input]
    return _levels(num_units, src, dst, allow_cycles=allow_cycles)


def _levels(n: int, src: np.ndarray, dst: np.ndarray, *, allow_cycles: bool) -> np.ndarray:
    levels = np.zeros(n, dtype=np.int64)
    if src.size == 0:
        return levels.astype(np.int32)
    by_dst = np.argsort(dst, kind="stable")
    s, d = src[by_dst], dst[by_dst]
    if _relax(levels, s, d, _QUICK_ROUNDS):
        return levels.astype(np.int32)
    # No fixpoint yet: a cycle, or a chain deeper than the quick rounds.
    tainted = _on_or_after_cycle(n, src, dst)
    if tainted.any() and not allow_cycles:
        raise ValueError("initial_levels: the edges contain a cycle (only a PIPELINE network may have one)")
    levels[:] = 0
    clean = ~tainted[s] & ~tainted[d]
    _relax(levels, s[clean], d[clean], n + 1)  # acyclic: settles within n + 1 rounds
    from_clean = ~tainted[s] & tainted[d]
    if from_clean.any():
        ts, td = s[from_clean], d[from_clean]
        starts = np.flatnonzero(np.r_[True, td[1:] != td[:-1]])
        levels[td[starts]] = np.maximum.reduceat(levels[ts], starts) + 1
    return levels.astype(np.int32)


def _relax(levels: np.ndarray, s: np.ndarray, d: np.ndarray, rounds: int) -> bool:
    """Raises levels[v] to max(levels[u] + 1) over the edges (u, v), sorted
    by v, until nothing changes (True) or `rounds` passes ran (False)."""
    if s.size == 0:
        return True
    starts = np.flatnonzero(np.r_[True, d[1:] != d[:-1]])
    heads = d[starts]
    for _ in range(rounds):
        cand = np.maximum.reduceat(levels[s], starts) + 1
        up = cand > levels[heads]
        if not up.any():
            return True
        levels[heads[up]] = cand[up]
    return False


def _on_or_after_cycle(n: int, src: np.ndarray, dst: np.ndarray) -> np.ndarray:
    """Units on a directed cycle (a strongly connected component of two or
    more units, or a self-loop) or reachable from one."""
    from scipy.sparse import csr_matrix
    from scipy.sparse.csgraph import breadth_first_order, connected_components

    ones = np.ones(src.size, dtype=np.int8)
    g = csr_matrix((ones, (src, dst)), shape=(n, n))
    ncomp, comp = connected_components(g, directed=True, connection="strong")
    on_cycle = np.bincount(comp, minlength=ncomp)[comp] > 1
    on_cycle[src[src == dst]] = True
    roots = np.flatnonzero(on_cycle)
    if roots.size == 0:
        return on_cycle
    # Breadth-first search from a virtual unit n with an edge to every root.
    s2 = np.concatenate([src, np.full(roots.size, n, dtype=np.int64)])
    d2 = np.concatenate([dst, roots])
    g2 = csr_matrix((np.ones(s2.size, dtype=np.int8), (s2, d2)), shape=(n + 1, n + 1))
    reached = np.zeros(n + 1, dtype=bool)
    reached[breadth_first_order(g2, n, directed=True, return_predecessors=False)] = True
    return reached[:n]


def capacity_policy(
    live: int,
    *,
    min_bucket: int = 64,
    headroom: float = 0.0,
    align: int | None = None,
) -> int:
    """Bucket capacity with headroom above the live count (topo.py:455-506):
    the next power of two (at least ``min_bucket``), or, with ``align``, a
    multiple of ``align``."""
    if headroom < 0.0:
        raise ValueError(f"capacity_policy: headroom must be >= 0, got {headroom}")
    if align is not None and align < 1:
        raise ValueError(f"capacity_policy: align must be >= 1, got {align}")
    target = math.ceil(max(live, 0) * (1.0 + headroom))
    if align is not None:
        target = max(target, min_bucket)
        return -(-target // align) * align
    if live <= 0:
        return min_bucket
    next_pow2 = 1 << (target - 1).bit_length()
    return max(next_pow2, min_bucket)


def resort(static, state):  # noqa: ANN001, ANN201 -- mirrors topo.resort
    """Recompute levels and lay the buckets out again on the device
    (topo.py:303-452); see plastax_amd.resort."""
    from plastax_amd.resort import resort as _resort

    return _resort(static, state)
