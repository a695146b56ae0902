"""Device unit lifecycle (update_unit, prune_unit, add_unit) against the
reference's unit goldens and the CPU oracle, bit for bit; the phases run on
the caller's unit numbering here (plastax_amd.units)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import unit_cases as uc
from oracle import growth as og
from plastax_amd import _site, grow, units as du
from plastax_amd.state import column_to_numpy, to_column

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _run_device(net, static, hu, hc):
    print(f"device unit phases: {net.__name__}", flush=True)
    uspecs = {s.name: s for s in static.unit_fields}
    cspecs = {s.name: s for s in static.conn_fields}
    units = {k: to_column(v, uspecs[k], DEV) for k, v in hu.items()}
    conns = [{k: to_column(v, cspecs[k], DEV) for k, v in b.items()} for b in hc]
    k = grow.Kernels(DEV, torch.cuda.current_stream(DEV).cuda_stream)
    pruned_by_phase: list[int] = []
    added, overflow = 0, False
    if net.update_unit is not None:
        du.UpdateUnitPhase(net, static, None).run(k, units, None)
    if net.prune_unit is not None:
        ph = du.PruneUnitPhase(net, static, None)
        doomed, count = ph.run(k, units, None)
        kills = torch.zeros(1, dtype=torch.int32, device=DEV)
        for b in conns:
            ph.kill_columns(k, int(b["dead"].shape[0]), b["from_id"], b["to_id"], b["dead"], doomed, kills)
        pruned_by_phase = np.flatnonzero(doomed.cpu().numpy()).tolist()
        assert int(count.item()) == len(pruned_by_phase)
    if net.add_unit is not None:
        added, overflow = du.AddUnitPhase(net, static, None).run(k, units, None)
    torch.cuda.synchronize()
    hu2 = {n: column_to_numpy(v, uspecs[n]) for n, v in units.items()}
    hc2 = [{n: column_to_numpy(v, cspecs[n]) for n, v in b.items()} for b in conns]
    return hu2, hc2, pruned_by_phase, added, overflow


def _run_oracle(net, static, hu, hc):
    dtypes = {s.name: np.dtype(s.dtype) for s in static.unit_fields}
    pruned_by_phase: list[int] = []
    added, overflow = 0, False
    if net.update_unit is not None:
        prog, names = _site.trace_update_unit(net.update_unit, dtypes, None)
        hu = og.update_unit(prog, names, hu, None)
    if net.prune_unit is not None:
        hu, hc, doomed = og.prune_unit(_site.trace_prune_unit(net.prune_unit, dtypes, None), static, hu, hc, None)
        pruned_by_phase = np.flatnonzero(doomed).tolist()
    if net.add_unit is not None:
        spawn = _site.trace_spawn(net.add_unit, dtypes, None)
        init, names = _site.trace_unit_init(net.add_unit, dtypes, None)
        hu, added, overflow, _ = og.add_unit(spawn, init, names, static, net.max_levels, hu, None)
    return hu, hc, pruned_by_phase, added, overflow


def _same(a: dict, b: dict) -> None:
    for name in a:
        x, y = np.asarray(a[name]), np.asarray(b[name])
        if x.dtype.kind == "f":
            assert np.array_equal(x.view(np.uint32), y.astype(x.dtype).view(np.uint32)), name
        else:
            assert np.array_equal(x.astype(np.int64), y.astype(np.int64)), name


@pytest.mark.parametrize("name", uc.UNIT_CASES)
def test_unit_golden_on_device(name: str) -> None:
    doc = uc.load(name)
    net = uc.golden_net(doc)
    static, hu, hc = uc.golden_state(net, doc)
    before = {k: v.copy() for k, v in hu.items()}
    got = _run_device(net, static, hu, hc)
    uc.check_against_golden(doc, before, *got)
    ref = _run_oracle(net, static, hu, hc)
    _same(got[0], ref[0])
    for b, r in zip(got[1], ref[1]):
        _same(b, r)
    assert got[2:] == ref[2:]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_unit_lifecycle_matches_oracle(seed: int) -> None:
    """A 5,000-slot net (4,000 allocated, some pruned): every unit phase,
    spawns that overflow the free slots (seed 2), deep offsets clamped."""
    rng = np.random.default_rng(seed)
    doc = {"rules": {"update_unit": "unit_update_v1", "prune_unit": "unit_prune_v1",
                     "add_unit": "unit_spawn_deep_v1" if seed == 1 else "unit_spawn_v1",
                     "init_unit": "unit_child_init_v1"},
           "capacity": 5000, "max_levels": 7}
    net = uc.golden_net(doc)
    n_alloc = 4000
    levels = rng.integers(0, 6, n_alloc)
    src = rng.integers(0, n_alloc, 20000)
    dst = rng.integers(0, n_alloc, 20000)
    keep = levels[dst] > levels[src]
    doc["initial_units"] = [
        {"id": int(i), "is_input": bool(i < 8), "is_output": bool(i >= n_alloc - 8), "level": int(levels[i]),
         "pruned": bool(rng.random() < 0.05), "fields": {"activation": float(np.float32(rng.standard_normal()))}}
        for i in range(n_alloc)]
    doc["initial_edges"] = [{"src": int(s), "dst": int(t), "fields": {"weight": 0.25}}
                            for s, t in zip(src[keep], dst[keep])]
    if seed == 2:  # more spawners than free slots
        doc["capacity"] = n_alloc + 10
    net = uc.golden_net(doc)
    import plastax_amd as px
    units = doc["initial_units"]
    edges = doc["initial_edges"]
    static, state = px.NetworkBuilder.from_edges(
        net, n_alloc, np.asarray([e["src"] for e in edges], np.int32), np.asarray([e["dst"] for e in edges], np.int32),
        weights=np.full(len(edges), 0.25, np.float32), input_ids=list(range(8)),
        output_ids=list(range(n_alloc - 8, n_alloc)), globals_=None, device="cpu")
    uspecs = {s.name: s for s in static.unit_fields}
    cspecs = {s.name: s for s in static.conn_fields}
    hu = {k: column_to_numpy(v, uspecs[k]).copy() for k, v in state.units.items()}
    hc = [{k: column_to_numpy(v, cspecs[k]).copy() for k, v in b.items()} for b in state.conns]
    hu["activation"][:n_alloc] = [u["fields"]["activation"] for u in units]
    hu["pruned"][:n_alloc] = [u["pruned"] for u in units]
    got = _run_device(net, static, hu, hc)
    ref = _run_oracle(net, static, hu, hc)
    _same(got[0], ref[0])
    for b, r in zip(got[1], ref[1]):
        _same(b, r)
    assert got[2:] == ref[2:]
    assert got[3] > 0
