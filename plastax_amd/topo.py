"""Host-side topology helpers: initial levels and bucket capacities.

Restates src/plastax/topo.py:35-130 (longest-path levels by a frontier Kahn
walk, inputs pinned to level 0) and topo.py:455-506 (capacity_policy).
"""

from __future__ import annotations

import math

import numpy as np


def initial_levels(
    num_units: int,
    edges: np.ndarray,
    *,
    allow_cycles: bool = False,
    input_ids: tuple[int, ...] = (),
) -> np.ndarray:
    """Longest-path levels: in-degree-0 units are level 0, level(v) = max over
    incoming (u -> v) of level(u) + 1 (topo.py:35-130).

    Edges into an input do not raise its level (but count for the cycle
    check). Raises ValueError on a cycle unless ``allow_cycles``, in which
    case cycle units keep the best level their acyclic predecessors reach.
    """
    edges = np.asarray(edges, dtype=np.int64).reshape(-1, 2)
    if input_ids and edges.shape[0]:
        into_input = np.isin(edges[:, 1], np.asarray(input_ids))
        if into_input.any():
            if not allow_cycles:
                initial_levels(num_units, edges)
            return initial_levels(num_units, edges[~into_input], allow_cycles=allow_cycles)
    levels = np.zeros(num_units, dtype=np.int32)
    if edges.shape[0] == 0:
        return levels
    src = edges[:, 0]
    dst = edges[:, 1]
    remaining = np.bincount(dst, minlength=num_units).astype(np.int64)
    settled = remaining == 0
    newly = settled.copy()
    processed = int(settled.sum())
    rounds = 0
    while bool(newly.any()):
        active = newly[src]
        active_dst = dst[active]
        levels[active_dst] = np.int32(rounds + 1)
        remaining -= np.bincount(active_dst, minlength=num_units)
        reached = (remaining == 0) & ~settled
        settled |= reached
        newly = reached
        processed += int(reached.sum())
        rounds += 1
    if processed != num_units and not allow_cycles:
        raise ValueError("initial_levels: edges do not form a DAG (cycle detected)")
    return levels


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
