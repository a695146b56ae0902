"""The churn layout's merged rebuild (ChurnArena with ``prev``: survivors
merged with the claimed slots by plx_merge_index / plx_merge_gather) must
give the full rebuild's arena entry for entry: every column over the whole
buffer (live range and the fill values past it), the live counts and, over
the live range, the slot map, the forward rows and the backward lists,
after every growth step,
with prunes that free slots the growth then claims again. Two identical
states step side by side, one per mode; both also match the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import c5_recipe as c5
import nets
import plastax_amd as px
from test_gpu_churn import Propose, TauPrune, _net
from test_gpu_parity import assert_same_state

pytestmark = pytest.mark.gpu


def _arrays(arena) -> dict[str, np.ndarray]:
    """Every column over the whole buffer; per bucket the live count, the
    slot map and the lists over the live range (a merged arena sizes its
    launches by a bound: past the count its lists and slot map hold fill
    values, the full build's slot map the dead slots)."""
    out = {f"col/{name}": col.cpu().numpy() for name, col in arena.cols.items()}
    lives = arena.live_counts()
    out["lives"] = np.asarray(lives)
    slot = arena.slot.cpu().numpy()
    for b, (f, lst) in enumerate(zip(arena.fwd, arena.lists)):
        live = lives[b]
        assert live <= arena.lives[b]
        out[f"slot{b}"] = slot[arena.bases[b] : arena.bases[b] + live]
        out[f"fwd{b}/ptr"] = f.ptr.cpu().numpy()
        out[f"list{b}/ptr"] = lst.ptr.cpu().numpy()
        out[f"list{b}/pos"] = lst.pos[: live + 1].cpu().numpy()
        out[f"list{b}/dst"] = lst.dst[: live + 1].cpu().numpy()
        out[f"list{b}/src"] = lst.src[:live].cpu().numpy()
        out[f"list{b}/slot"] = lst.slot[:live].cpu().numpy()
    return out


def _same(a: dict, b: dict, what: str) -> None:
    assert a.keys() == b.keys(), what
    for key in a:
        x, y = a[key], b[key]
        same = x.shape == y.shape and (np.array_equal(x.view(np.uint32), y.view(np.uint32)) if x.dtype == np.float32
                                       else np.array_equal(x, y))
        assert same, f"{what}: {key} differs"


def _lockstep(oracle, net, build, steps: int, globals_fn, inputs_fn, check_every: int = 1) -> int:
    runs = []
    for mode in ("merge", "full"):
        static, state = build()
        step = px.make_step(net, static)
        step.relayout = mode
        runs.append([static, state, step])
    static0 = runs[0][0]
    o = nets.oracle_for(oracle, net, static0, runs[0][1])
    o.tail_start, o.needs_resort = int(runs[0][1].tail_start), bool(runs[0][1].needs_resort)
    assert runs[0][2].backward_order == "slot"
    o.tile = None
    merged = 0
    for k in range(1, steps + 1):
        g = globals_fn(k)
        x, t = inputs_fn(k)
        print(f"merge-relayout step {k}", flush=True)
        for run in runs:
            run[1].globals_ = g
            run[1] = run[2](run[1], px.StepInputs(x, t)).state
        o.globals_ = g
        o.step(x, t) if t is not None else o.step(x)
        st_m, st_f = runs[0][1], runs[1][1]
        assert (st_m.grown, st_m.units_added) == (st_f.grown, st_f.units_added) == (o.grown, o.units_added)
        # lay both out (the next step would): the merged one from its predecessor
        am = runs[0][2].arena(st_m)
        af = runs[1][2].arena(st_f)
        merged += int(am.merged)
        assert not af.merged
        if k % check_every == 0:
            torch.cuda.synchronize()
            _same(_arrays(am), _arrays(af), f"step {k}")
            assert_same_state(static0, st_m, o, f"step {k} (merge)")
    return merged


def test_reservoir_merged_relayout_equals_the_full_build(oracle) -> None:
    rng = np.random.default_rng(21)
    n = 1200
    src = rng.integers(0, n, 9000).astype(np.int32)
    dst = rng.integers(0, n, 9000).astype(np.int32)
    keep = src != dst
    src, dst = src[keep], dst[keep]
    w = (rng.standard_normal(src.size) * 0.3).astype(np.float32)
    net = _net(True, Propose(n), px.optim.adam(1e-2, nets.GRAD_PRE_ACT))

    def build():
        return px.NetworkBuilder.from_edges(
            net, n, src, dst, weights=w, input_ids=np.arange(32), output_ids=np.arange(n - 8, n),
            globals_={"tau": np.float32(0.0)}, capacity_headroom=1.0, device="cuda")

    drng = np.random.default_rng(3)
    xs = drng.standard_normal((13, 32)).astype(np.float32)
    ts = np.tanh(drng.standard_normal((13, 8))).astype(np.float32)
    # tau rises and falls: prunes free slots that later growth claims again
    merged = _lockstep(oracle, net, build, 12, lambda k: {"tau": np.float32(0.01 * (k % 4))},
                       lambda k: (xs[k], ts[k]))
    assert merged >= 10


def test_c5_recipe_merged_relayout_equals_the_full_build(oracle) -> None:
    """Unit prunes (PruneUnit of zero out-degree) kill edges inside the live
    range; AddUnit steps (every 5 steps here) fall back to the full build."""
    n, cap, n_in = 1024, 4096, 32
    net = c5.recipe(n_in, n, 128, 16, 8, cap)
    src, dst, w = c5.reservoir_edges(0, n, 48 * 1024, n_in)

    def build():
        return px.NetworkBuilder.from_edges(
            net, n, src, dst, weights=w, input_ids=np.arange(n_in), output_ids=np.arange(n - 8, n),
            globals_={"spawn": np.float32(0.0)}, capacity_headroom=1.0, device="cuda")

    drng = np.random.default_rng(4)
    xs = drng.standard_normal((31, n_in)).astype(np.float32)
    merged = _lockstep(oracle, net, build, 30, lambda k: {"spawn": np.float32(1.0 if k % 5 == 0 else 0.0)},
                       lambda k: (xs[k], None), check_every=3)
    assert merged >= 20
