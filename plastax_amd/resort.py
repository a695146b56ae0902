"""topo.resort on the device: recompute the levels from the live edges and
lay the buckets out again (topo.py:189-452).

- ``has_cycle`` (topo.py:253-301): longest-path relaxation over the live
  edges with no unit pinned, until a round changes nothing (acyclic) or
  ``num_units`` rounds have all changed something (a cycle);
- ``recompute_levels`` (topo.py:189-251): the same relaxation from all-zero
  levels with the declared inputs pinned to 0 after every round, for
  ``kahn_max_depth`` (or ``num_units``) rounds -- stopping at the first round
  that changes nothing gives the same levels;
- ``resort`` (topo.py:303-452): every live edge goes to the bucket of its
  source's new level (one bucket for PIPELINE), keeping its old relative
  order and then sorted stably by source; new capacities are
  ``max(capacity_policy(live), old capacity)``.

Rounds run in batches on the stream with one flag read per batch.
"""

from __future__ import annotations

import dataclasses
from typing import Any

import numpy as np
import torch

from plastax_amd import _lib
from plastax_amd._types import Propagation
from plastax_amd.grow import Kernels, _bits_for, flatten
from plastax_amd.state import NetworkState, NetworkStatic, to_column
from plastax_amd.topo import capacity_policy

_BATCH = 16


def _relax(k: Kernels, flat: dict, n: int, level: torch.Tensor, is_input: torch.Tensor | None,
           rounds_max: int) -> tuple[torch.Tensor, bool]:
    """Run up to ``rounds_max`` relaxation rounds; returns the levels and
    whether a round changed nothing (convergence)."""
    e = int(flat["dead"].shape[0])
    cur = level.clone()
    nxt = torch.empty_like(cur)
    done = 0
    while done < rounds_max:
        batch = min(_BATCH, rounds_max - done)
        changed = torch.zeros(batch, dtype=torch.int32, device=cur.device)
        for r in range(batch):
            _lib.check(k.lib.plx_relax_levels(n, e, flat["from_id"].data_ptr(), flat["to_id"].data_ptr(),
                                              flat["dead"].data_ptr(), cur.data_ptr(), nxt.data_ptr(),
                                              None if is_input is None else is_input.data_ptr(),
                                              changed[r:].data_ptr(), k.s), "plx_relax_levels")
            cur, nxt = nxt, cur
        flags = changed.cpu().numpy()
        if not flags.all():
            return cur, True  # converged: every later round is a no-op
        done += batch
    return cur, False


def _input_mask(static: NetworkStatic, device: torch.device) -> torch.Tensor:
    m = np.zeros(static.num_units, np.uint8)
    if static.input_ids:
        m[np.asarray(static.input_ids, dtype=np.int64)] = 1
    return torch.from_numpy(m).to(device)


def has_cycle(static: NetworkStatic, state: NetworkState, k: Kernels | None = None) -> bool:
    """Whether the live connections contain a directed cycle (topo.py:253-301)."""
    conns = state.conns
    flat, _ = flatten(conns)
    dev = flat["dead"].device
    k = k or Kernels(dev, int(torch.cuda.current_stream(dev).cuda_stream))
    n = static.num_units
    _, converged = _relax(k, flat, n, torch.zeros(n, dtype=torch.int32, device=dev), None, n)
    return not converged


def recompute_levels(static: NetworkStatic, state: NetworkState, k: Kernels | None = None) -> torch.Tensor:
    """Longest-path levels of the live edges, inputs pinned to 0 (topo.py:189-251)."""
    flat, _ = flatten(state.conns)
    dev = flat["dead"].device
    k = k or Kernels(dev, int(torch.cuda.current_stream(dev).cuda_stream))
    n = static.num_units
    depth = static.kahn_max_depth if static.kahn_max_depth is not None else n
    level, _ = _relax(k, flat, n, torch.zeros(n, dtype=torch.int32, device=dev), _input_mask(static, dev), depth)
    return level


def resort(static: NetworkStatic, state: NetworkState) -> tuple[NetworkStatic, NetworkState]:
    """Recompute the levels and lay the buckets out again (topo.py:303-452).
    Raises ValueError for a TOPOLOGICAL net whose live edges hold a cycle."""
    conns = state.conns
    units = dict(state.units)
    flat, offs = flatten(conns)
    dev = flat["dead"].device
    k = Kernels(dev, int(torch.cuda.current_stream(dev).cuda_stream))
    n = static.num_units
    pipeline = static.propagation is Propagation.PIPELINE
    if not pipeline:
        _, converged = _relax(k, flat, n, torch.zeros(n, dtype=torch.int32, device=dev), None, n)
        if not converged:
            raise ValueError(
                "resort: topological propagation requires an acyclic graph; the live connections contain a cycle"
            )
    depth = static.kahn_max_depth if static.kahn_max_depth is not None else n
    new_level, _ = _relax(k, flat, n, torch.zeros(n, dtype=torch.int32, device=dev), _input_mask(static, dev), depth)
    if pipeline:
        nb = 1
    else:
        max_level = int(new_level.max().item()) if n else 0
        nb = max(max_level + (1 if static.deepest_grows else 0), 1)
    total = offs[-1]
    keys = k.mem.i32(total)
    _lib.check(k.lib.plx_resort_keys(total, flat["from_id"].data_ptr(), flat["dead"].data_ptr(),
                                     new_level.data_ptr(), int(pipeline), nb, keys.data_ptr(), k.s),
               "plx_resort_keys")
    count, start = k.mem.i32(nb), k.mem.i32(nb)
    scratch = k.mem.ints_for(nb)
    _lib.check(k.lib.plx_level_counts(total, None, keys.data_ptr(), nb, count.data_ptr(), start.data_ptr(),
                                      scratch.data_ptr(), k.s), "plx_level_counts")
    order, nlive = k.compact(total, 1, flat["dead"])  # the live slots, in flat order
    k.sort(order, total, [(0, _bits_for(n), flat["from_id"], None), (0, _bits_for(nb), keys, None)], n_dev=nlive)
    live_counts = count.cpu().numpy().astype(np.int64).tolist()
    starts = start.cpu().numpy().astype(np.int64).tolist()
    old_caps = static.level_capacities
    caps = tuple(
        max(capacity_policy(live, headroom=static.capacity_headroom, align=static.capacity_align),
            old_caps[b] if b < len(old_caps) else 0)
        for b, live in enumerate(live_counts)
    )
    specs = {s.name: s for s in static.conn_fields}
    new_conns = []
    for b in range(nb):
        cols = {}
        for name, spec in specs.items():
            col = to_column(np.full((caps[b],), spec.default, dtype=spec.dtype), spec, dev)
            if live_counts[b]:
                _lib.check(k.lib.plx_gather_col(live_counts[b], None, order[starts[b]:].data_ptr(),
                                                flat[name].data_ptr(), col.data_ptr(), col.element_size(), k.s),
                           "plx_gather_col")
            cols[name] = col
        new_conns.append(cols)
    units["level"] = new_level
    new_static = dataclasses.replace(static, level_capacities=caps)
    new_state = NetworkState(
        units, tuple(new_conns), state.globals_, False, state.step, state.grown, state.overflow,
        state.units_added, state.unit_overflow, live_counts[0] if pipeline else 0,
    )
    state._donated = True
    return new_static, new_state
