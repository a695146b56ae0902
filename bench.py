"""Benchmark of the streaming edge-arena step (forward + backward + update).

Default workload: configuration C2 -- 8 layers x 131,072 tanh units, 2^26
edges with Zipf(1.1) source popularity, MSE to a signed-permutation target,
Adam(1e-3), batch 1 streaming -- on one MI355X. Inputs and targets for every
step are generated up front and resident in HBM before the timed region.

Prints one JSON line: edges/s over the timed steps (live edges / step time),
the roofline of the dominant kernel (algorithmic bytes per launch / mean launch
time from HIP events recorded on the launching stream inside the timed
region), and the CPU oracle timed on the host on a bounded sample.
"""

from __future__ import annotations

import argparse
import collections
import json
import os
import pathlib
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
# C2: the default timed steps, and the pool of synthetic samples the steps
# cycle through (step k streams sample k % pool)
C2_DEFAULT_STEPS = 6000
C2_INPUT_POOL = 1000


def progress(msg: str) -> None:
    """A setup/progress line on stderr (stdout carries only the JSON line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


METRIC = "edges/sec per streaming step (fwd+bwd+update) at 64M edges; % of HBM peak"


class EventTimer:
    """HIP events around kernel launches, on torch's current stream (the
    stream every launch of the step goes to). ``kinds`` limits the recording
    to those launch kinds; with ``stride`` only every stride-th launch of a
    kind is bracketed (an event pair costs the stream a few microseconds),
    and each recorded launch keeps its ordinal among the kind's launches."""

    def __init__(self, kinds: set[str] | None = None, stride: int = 1) -> None:
        import torch

        self.torch = torch
        self.on = False
        self.kinds = kinds
        self.stride = max(1, int(stride))
        self.count: dict[str, int] = collections.defaultdict(int)
        self.pairs: dict[str, list] = collections.defaultdict(list)
        self._open: tuple | None = None

    def begin(self, kind: str) -> None:
        if self.on and (self.kinds is None or kind in self.kinds):
            c = self.count[kind]
            self.count[kind] = c + 1
            if c % self.stride:
                return
            e = self.torch.cuda.Event(enable_timing=True)
            e.record()
            self._open = (kind, e, c)

    def end(self, kind: str) -> None:
        if self.on and self._open is not None:
            e = self.torch.cuda.Event(enable_timing=True)
            e.record()
            self.pairs[kind].append((self._open[1], e, self._open[2]))
            self._open = None

    def summary(self) -> dict[str, dict]:
        self.torch.cuda.synchronize()
        out = {}
        for kind, pairs in self.pairs.items():
            ms = [a.elapsed_time(b) for a, b, _ in pairs]
            out[kind] = {"launches": len(ms), "total_ms": float(sum(ms)), "mean_ms": float(np.mean(ms)),
                         "ms": ms, "ordinals": [c for _, _, c in pairs]}
        return out


def kernel_table(kernels: dict[str, dict]) -> dict[str, dict]:
    """The breakdown as printed: launches, total and mean ms per kind."""
    return {k: {"launches": v["launches"], "total_ms": round(v["total_ms"], 3), "mean_ms": round(v["mean_ms"], 4)}
            for k, v in kernels.items()}


def build_c2(px, seed: int, scale: int):
    import plastax_amd.numpy as jnp
    from plastax_amd import synth

    grad = px.FieldSpec.float32("grad_pre_act")
    lossg = px.FieldSpec.float32("loss_grad")

    class TanhForward(px.ForwardPass):
        combine = px.monoid.sum_

        def map(self, u, dst, src, c, cid, g):
            return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)))

    class TanhBackward(px.BackwardPass):
        combine = px.monoid.sum_

        def map(self, u, src, dst, c, cid, g):
            return c[px.WEIGHT, cid] * u[grad, dst]

        def apply(self, u, i, g, acc):
            a = u[px.ACTIVATION, i]
            return px.UnitWrite.of((grad, (acc + u[lossg, i]) * (jnp.float32(1.0) - a * a)))

    class MSELoss(px.Loss):
        seed_field = lossg

        def calculate_loss(self, u, outputs, targets, g):
            d = u.gather(px.ACTIVATION, outputs) - targets
            return jnp.sum(jnp.float32(0.5) * d * d), d

    opt = px.optim.adam(1e-3, grad)

    class C2Net(px.Network):
        forward_pass = TanhForward()
        backward_pass = TanhBackward()
        loss = MSELoss()
        update_conn = opt.update_conn()
        extra_unit_fields = (grad, lossg)
        extra_conn_fields = opt.state_fields
        propagation = px.Propagation.TOPOLOGICAL

    e = synth.c2_topological(seed=seed, scale=scale)
    return C2Net, e


def host_cpu() -> dict:
    """The host's CPU model and counts (the CPU baseline runs on these cores)."""
    model = None
    try:
        for line in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def cpu_baseline(px, net, static, e, host_units, host_conns, inputs, targets, steps: int) -> dict:
    """The oracle (the C restatement, -O3, OpenMP) on the same workload, timed
    twice from the same initial state: one thread in its sequential form, and
    all the threads OpenMP is given in its parallel form (the same folds, so
    the same bits: both legs' losses are returned for the parity check)."""
    from oracle import oracle as ox
    from plastax_amd._plan import compile_plan

    plan = compile_plan(net, static)
    legs = {}
    for name, parallel in (("single_thread", False), ("all_cores", True)):
        o = ox.OracleNet(static, {k: v.copy() for k, v in host_units.items()},
                         [{k: v.copy() for k, v in b.items()} for b in host_conns], plan, parallel=parallel)
        threads = o.lib.ox_set_threads(1 if not parallel else max(1, len(os.sched_getaffinity(0))))
        if parallel and os.environ.get("OMP_NUM_THREADS"):
            threads = o.lib.ox_set_threads(int(os.environ["OMP_NUM_THREADS"]))
        losses = [np.float32(o.step(inputs[0], targets[0]))]  # warm-up
        times = []
        for k in range(steps):
            t0 = time.perf_counter()
            losses.append(np.float32(o.step(inputs[(k + 1) % len(inputs)], targets[(k + 1) % len(targets)])))
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        legs[name] = {"value": float(e.src.size / med), "cores": int(threads), "median_step_ms": round(med * 1e3, 1),
                      "losses": losses}
        del o
        o = None
        progress(f"CPU baseline ({name}, {threads} thread(s)): {med * 1e3:.1f} ms per C2 step")
    one, allc = legs["single_thread"], legs["all_cores"]
    return {
        "losses": {k: v.pop("losses") for k, v in legs.items()},
        "value": allc["value"],
        "unit": "edges/s",
        "cores": allc["cores"],
        "kind": "port",
        "sample": f"{steps} full C2 steps ({e.src.size} edges) after 1 warm-up, median step "
        f"{allc['median_step_ms']} ms on {allc['cores']} threads; the C oracle (oracle/plastax_oracle.c, "
        "gcc -O3 -march=x86-64-v3 -fopenmp, no contraction), its parallel form",
        "single_thread": {"value": one["value"], "cores": 1, "median_step_ms": one["median_step_ms"],
                          "form": "sequential (slot-order loops)"},
        "host": host_cpu(),
    }


GROWTH_METRIC = "add_conn proposals/sec per growth phase (C5 reservoir, per-unit ProposeAddConn, P=4)"


def build_c5(px):
    """C5's growing reservoir at its starting shape, with the per-unit
    proposal rule of the configuration (P = 4 via the counter-based rng)."""
    import plastax_amd.numpy as jnp

    class Tanh(px.ForwardPass):
        combine = px.monoid.sum_

        def map(self, u, dst, src, c, cid, g):
            return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)))

    class Propose(px.ProposeAddConn):
        proposer = "per_unit"
        proposals_per_proposer = 4
        max_new_per_level = 16
        max_level_gap = 1 << 20

        def propose(self, u, i, j, g, rng):
            dst = rng.uniform_int(65536).astype(jnp.int32)
            return jnp.asarray(i, jnp.int32), dst, rng.uniform()

        def init(self, u, src, dst, g):
            return px.ConnWrite.of((px.WEIGHT, jnp.float32(0.01)))

    class C5(px.Network):
        forward_pass = Tanh()
        add_conn = Propose()
        propagation = px.Propagation.PIPELINE
        unit_capacity = 262144

    return C5


def run_c5_growth(args) -> int:
    """The add_conn phase of C5 on the device: 262,144 unit slots x 4
    proposals per phase, over the 16M-slot logical arena; each timed phase
    commits its winners, so the arena evolves like C5's every-step growth."""
    import torch

    import plastax_amd as px
    from plastax_amd import grow, synth
    from plastax_amd.state import column_to_numpy

    t_setup = time.perf_counter()
    net = build_c5(px)
    e = synth.c5_reservoir(args.seed)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, capacity_headroom=3.0, device="cpu")
    progress(f"C5 arena: {e.src.size} live edges of {static.level_capacities[0]} slots "
             f"({time.perf_counter() - t_setup:.1f} s)")
    uspecs = {s.name: s for s in static.unit_fields}
    cspecs = {s.name: s for s in static.conn_fields}
    host_units = {k: column_to_numpy(v, uspecs[k]).copy() for k, v in state.units.items()}
    host_conns = [{k: column_to_numpy(v, cspecs[k]).copy() for k, v in b.items()} for b in state.conns]
    tail0 = int(state.tail_start)
    dev = torch.device("cuda", 0)
    units = {k: v.to(dev) for k, v in state.units.items()}
    conns = tuple({k: v.to(dev) for k, v in b.items()} for b in state.conns)
    phase = grow.AddConnPhase(net, static, None)
    timer = EventTimer({"total_order"})
    k = grow.Kernels(dev, torch.cuda.current_stream(dev).cuda_stream, timer=timer)
    tail = tail0
    for it in range(args.warmup):
        out = phase.run(k, units, conns, step=it, globals_=None, tail_start=tail)
        conns, tail = out.conns, out.tail_start
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup
    timer.on = True
    grown = 0
    t0 = time.perf_counter()
    for it in range(args.warmup, args.warmup + args.steps):
        out = phase.run(k, units, conns, step=it, globals_=None, tail_start=tail)
        conns, tail = out.conns, out.tail_start
        grown += out.grown
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    timer.on = False
    dom = timer.summary()["total_order"]
    n_sorted = int(phase.last_sort[0].item())
    passes = int(phase.last_sort[1])
    sites = int(static.num_units) * 4
    ms = elapsed * 1e3 / args.steps
    # The total order's radix passes read and write each key and index once
    # (16 B per sorted candidate per 8-bit pass).
    per_launch = 16 * passes * n_sorted
    ach = per_launch / (dom["mean_ms"] * 1e-3) / 1e9
    roofline = {
        "kernel": "total_order (plx_sort)",
        "bound": "hbm",
        "achieved": round(ach, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(ach / HBM_PEAK_GBS, 4),
        "traffic": None,
        "algorithmic_bytes_per_launch": per_launch,
        "mean_launch_ms": round(dom["mean_ms"], 4),
    }
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import growth as og

        times = []
        tail_c = tail0
        conns_c = host_conns
        for it in range(1):
            t1 = time.perf_counter()
            res = og.add_conn(net, static, host_units, conns_c, step=it, globals_=None, tail_start=tail_c)
            times.append(time.perf_counter() - t1)
            conns_c, tail_c = res.conns, res.tail_start
        med = float(np.median(times))
        cpu = {
            "value": float(sites / med),
            "unit": "proposals/s",
            "cores": 1,
            "kind": "port",
            "sample": f"1 add_conn phase of the same workload, {med * 1e3:.0f} ms "
            "(numpy + the C site interpreter of oracle/, one thread)",
        }
    line = {
        "metric": GROWTH_METRIC,
        "value": round(sites / (ms * 1e-3), 1),
        "unit": "proposals/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic",
        "config": {
            "workload": "C5 growth phase: 65,536 live of 262,144 unit slots, 4M live of 16M edge slots, "
            "PIPELINE, per-unit proposals P=4, max_new_per_level 16",
            "sites": sites,
            "sorted_candidates": n_sorted,
            "radix_passes": passes,
        },
        "grown_per_phase": grown / args.steps,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(line), flush=True)
    return 0


C5_METRIC = ("steps/sec of C5's growing reservoir (forward + out-degree count + PruneUnit + AddUnit + "
             "per-unit proposals + growth + device relayout)")


def build_c5_recipe(px, num_units: int, unit_capacity: int, spawn_lo: int, spawn_n: int):
    """C5's recipe: the PIPELINE tanh reservoir, a backward pass that counts
    every unit's live out-edges (a constant map under sum_), PruneUnit of the
    units whose out-degree is zero, AddUnit spawning the parents with ids in
    [spawn_lo, spawn_lo + spawn_n) when the global ``spawn`` is set (the bench
    sets it every 100 steps), and per-unit proposals (P = 4, counter-based
    rng) every step."""
    import plastax_amd.numpy as jnp

    outdeg = px.FieldSpec.float32("out_degree")

    class Tanh(px.ForwardPass):
        combine = px.monoid.sum_

        def map(self, u, dst, src, c, cid, g):
            return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)))

    class CountOut(px.BackwardPass):
        combine = px.monoid.sum_

        def map(self, u, src, dst, c, cid, g):
            return jnp.float32(1.0)

        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((outdeg, acc))

    class PruneSilent(px.PruneUnit):
        def predicate(self, u, i, g):
            return u[outdeg, i] == jnp.float32(0.0)

    class SpawnBand(px.AddUnit):
        def spawn(self, u, parent, g):
            band = (parent >= spawn_lo) & (parent < spawn_lo + spawn_n)
            return band & (g["spawn"] > jnp.float32(0.0)), jnp.int32(0)

        def init(self, u, child, parent, g):
            return px.UnitWrite.of((px.ACTIVATION, u[px.ACTIVATION, parent] * jnp.float32(0.5)))

    class Propose(px.ProposeAddConn):
        proposer = "per_unit"
        proposals_per_proposer = 4
        max_new_per_level = 16
        max_level_gap = 1 << 20

        def propose(self, u, i, j, g, rng):
            dst = rng.uniform_int(num_units).astype(jnp.int32)
            return jnp.asarray(i, jnp.int32), dst, rng.uniform()

        def init(self, u, src, dst, g):
            return px.ConnWrite.of((px.WEIGHT, jnp.float32(0.01)))

    class C5(px.Network):
        unit_capacity = 262144
        forward_pass = Tanh()
        backward_pass = CountOut()
        prune_unit = PruneSilent()
        add_unit = SpawnBand()
        add_conn = Propose()
        extra_unit_fields = (outdeg,)
        propagation = px.Propagation.PIPELINE

    C5.unit_capacity = unit_capacity
    return C5


def run_c5(args) -> int:
    """C5 end to end, its whole recipe: every step scatters 256 inputs, runs
    the PIPELINE forward and the out-degree count over the live edges, prunes
    the units left without out-edges, spawns 16 units every 100 steps, grows
    (per-unit proposals, P = 4), and the next step lays the arena out again on
    the device (the churn layout). The first steps are checked against the
    oracle from the same initial state: flags every step and, after them,
    every unit and connection column bit for bit."""
    import torch

    import plastax_amd as px
    from plastax_amd import synth
    from plastax_amd.state import column_to_numpy

    t_setup = time.perf_counter()
    e = synth.c5_reservoir(args.seed)
    net = build_c5_recipe(px, e.num_units, 262144, 1024, 16)
    g_of = lambda k: {"spawn": np.float32(1.0 if k % 100 == 0 else 0.0)}  # noqa: E731
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=g_of(0), capacity_headroom=3.0, device="cpu")
    uspecs = {s.name: s for s in static.unit_fields}
    cspecs = {s.name: s for s in static.conn_fields}
    host_units = {k: column_to_numpy(v, uspecs[k]).copy() for k, v in state.units.items()}
    host_conns = [{k: column_to_numpy(v, cspecs[k]).copy() for k, v in b.items()} for b in state.conns]
    dev = torch.device("cuda", 0)
    gstate = px.NetworkState(
        {k: v.to(dev) for k, v in state.units.items()},
        tuple({k: v.to(dev) for k, v in b.items()} for b in state.conns),
        g_of(0),
    )
    gstate.tail_start = state.tail_start
    step = px.make_step(net, static)
    step.relayout = args.relayout
    npar = 0 if args.no_cpu_baseline else 2
    nsteps = npar + args.warmup + args.steps
    rng = np.random.default_rng(args.seed + 3)
    xs = rng.standard_normal((nsteps, e.input_ids.size)).astype(np.float32)
    xs_d = torch.from_numpy(xs).to(dev)
    flags = []
    k = 0
    for _ in range(npar):
        gstate.globals_ = g_of(k)
        gstate = step(gstate, px.StepInputs(xs_d[k])).state
        flags.append((int(gstate.units_added), bool(gstate.unit_overflow), int(gstate.grown),
                      bool(gstate.overflow), int(gstate.tail_start)))
        k += 1
    snap = None
    if npar:
        torch.cuda.synchronize()
        snap = ({n: column_to_numpy(gstate.units[n], uspecs[n]).copy() for n in uspecs},
                [{n: column_to_numpy(b[n], cspecs[n]).copy() for n in cspecs} for b in gstate.conns])
    for _ in range(args.warmup):
        gstate.globals_ = g_of(k)
        gstate = step(gstate, px.StepInputs(xs_d[k])).state
        k += 1
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup
    progress(f"C5: {e.src.size} live edges of {static.level_capacities[0]} slots, layout {step.backward_order} "
             f"({setup_s:.1f} s)")
    # Each step's flags stay on the device; they are read after the timed
    # region (a driver checking them every step would add a host read per
    # step on top of the step itself).
    readers = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        gstate.globals_ = g_of(k)
        gstate = step(gstate, px.StepInputs(xs_d[k])).state
        readers.append((gstate._flag_reader("grown"), gstate._flag_reader("units_added")))
        k += 1
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    grown = sum(int(r()) for r, _ in readers)
    added = sum(int(r()) for _, r in readers)
    ms = elapsed * 1e3 / args.steps
    live = int(sum(int((b["dead"] == 0).sum().item()) for b in gstate.conns))
    live_units = int((gstate.units["pruned"] == 0).sum().item())
    cpu = None
    parity = None
    if npar:
        from oracle import oracle as ox
        from plastax_amd._plan import compile_plan

        ox.load()
        o = ox.OracleNet(static, host_units, host_conns, compile_plan(net, static), g_of(0), tile=None)
        o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
        times = []
        same_flags = True
        for q in range(npar):
            o.globals_ = g_of(q)
            t1 = time.perf_counter()
            o.step(xs[q])
            times.append(time.perf_counter() - t1)
            same_flags &= flags[q] == (o.units_added, o.unit_overflow, o.grown, o.overflow, o.tail_start)
        units_d, conns_d = snap
        same_units = all(np.array_equal(units_d[n].view(np.uint8), o.units[n].view(np.uint8)) for n in uspecs)
        same_conns = all(np.array_equal(conns_d[b][n].view(np.uint8), o.conns[b][n].view(np.uint8))
                         for b in range(len(conns_d)) for n in cspecs)
        parity = {"steps": npar, "flags_equal": bool(same_flags), "units_bit_exact": bool(same_units),
                  "conns_bit_exact": bool(same_conns), "spawn_step_included": True}
        progress(f"C5 parity over {npar} steps: flags {same_flags}, units {same_units}, conns {same_conns}")
        sec = float(np.median(times))
        cpu = {
            "value": float(1.0 / sec),
            "unit": "steps/s",
            "cores": 1,
            "kind": "port",
            "sample": f"{npar} full C5 recipe steps of the same workload (the first spawns 16 units), median "
            f"{sec:.2f} s, the C oracle and oracle/growth.py, one thread",
        }
    line = {
        "metric": C5_METRIC,
        "value": round(1e3 / ms, 2),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "C5: 65,536 live of 262,144 unit slots, 4M live of 16M edge slots, PIPELINE tanh, "
            "out-degree count, PruneUnit (zero out-degree), AddUnit 16 per 100 steps, per-unit proposals "
            "P=4 every step, max_new_per_level 16",
            "layout": step.backward_order,
            "live_edges_end": live,
            "live_units_end": live_units,
        },
        "grown_per_step": grown / args.steps,
        "units_added": added,
        "roofline": None,
        "cpu_baseline": cpu,
        "full_size_parity": parity,
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(line), flush=True)
    return 0


C4_METRIC = "steps/sec of C4's dynamic sparse training (C3's sparse MLP at batch 1, prune + regrow every 100 steps)"


def build_c4(px):
    """C4: C3's sparse MLP at batch 1 with tanh units (their gradients stay
    alive, so regrowth scores are not all zero), softmax cross-entropy,
    Adam(1e-3); every 100 steps a PruneConn drops the live edges with |w|
    below the global tau (the driver sets it to the 10th percentile of the
    live |w|) and a ScoreAddConn regrows up to 1,024 edges per level from a
    32 x 32 shortlist scored by |act[src] * grad[dst]|."""
    import plastax_amd.numpy as jnp

    grad = px.FieldSpec.float32("grad_pre_act")
    lossg = px.FieldSpec.float32("loss_grad")

    class Tanh(px.ForwardPass):
        combine = px.monoid.sum_

        def map(self, u, dst, src, c, cid, g):
            return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)))

    class TanhBack(px.BackwardPass):
        combine = px.monoid.sum_

        def map(self, u, src, dst, c, cid, g):
            return c[px.WEIGHT, cid] * u[grad, dst]

        def apply(self, u, i, g, acc):
            a = u[px.ACTIVATION, i]
            return px.UnitWrite.of((grad, (acc + u[lossg, i]) * (jnp.float32(1.0) - a * a)))

    class MagnitudePrune(px.PruneConn):
        def predicate(self, u, c, cid, g):
            return jnp.abs(c[px.WEIGHT, cid]) < g["tau"]

    class GradGrow(px.ScoreAddConn):
        candidates = "shortlist_per_level"
        shortlist_size = 32
        direction = "deeper"
        max_level_gap = 1
        dedupe_live = True
        max_new_per_level = 1024
        trigger = ("every", 100)

        def score(self, u, src, dst, g):
            return jnp.abs(u[px.ACTIVATION, src] * u[grad, dst])

        def importance(self, u, i, g):
            return jnp.abs(u[grad, i]) + jnp.abs(u[px.ACTIVATION, i])

        def init(self, u, src, dst, g):
            return px.ConnWrite.of((px.WEIGHT, jnp.float32(0.0)))

    opt = px.optim.adam(1e-3, grad)

    class C4Net(px.Network):
        forward_pass = Tanh()
        backward_pass = TanhBack()
        loss = px.SoftmaxCrossEntropyLoss(lossg)
        update_conn = opt.update_conn()
        prune_conn = MagnitudePrune()
        add_conn = GradGrow()
        extra_unit_fields = (grad, lossg)
        extra_conn_fields = tuple(opt.state_fields)

    return C4Net


def run_c4(args) -> int:
    """C4 end to end: all 5,000 batch-1 steps (--c4-steps) from the built
    state, a prune + regrow event every 100 steps (steps 1, 101, ...). The
    driver sets tau, the 10th percentile of the live |w|, before each event
    step (one host read per 100 steps, outside the step). The first two
    steps (an event step and a plain one) run again from the same state
    against the oracle: flags, loss and every unit and connection column,
    bit for bit; their oracle time is the CPU leg."""
    import torch

    import plastax_amd as px
    from plastax_amd import synth
    from plastax_amd.state import column_to_numpy

    t_setup = time.perf_counter()
    net = build_c4(px)
    e = synth.c3_mlp(args.seed)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids, output_ids=e.output_ids,
        globals_={"tau": np.float32(0.0)}, capacity_headroom=0.1, device="cpu")
    uspecs = {s.name: s for s in static.unit_fields}
    cspecs = {s.name: s for s in static.conn_fields}
    host_units = {k: column_to_numpy(v, uspecs[k]).copy() for k, v in state.units.items()}
    host_conns = [{k: column_to_numpy(v, cspecs[k]).copy() for k, v in b.items()} for b in state.conns]
    dev = torch.device("cuda", 0)

    def fresh():
        return px.NetworkState({k: v.to(dev) for k, v in state.units.items()},
                               tuple({k: v.to(dev) for k, v in b.items()} for b in state.conns),
                               {"tau": np.float32(0.0)})

    def live_tau(st) -> np.float32:
        w = torch.cat([b["weight"][b["dead"] == 0].abs() for b in st.conns])
        return np.float32(torch.quantile(w, 0.1).item())

    nsteps = args.c4_steps
    xs, ys = synth.c3_batches(args.seed + 1, nsteps, 1)
    xs_d, ys_d = torch.from_numpy(xs[:, 0]).contiguous().to(dev), torch.from_numpy(ys[:, 0]).contiguous().to(dev)
    step = px.make_step(net, static)
    gstate = fresh()
    step.arena(gstate)
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup
    progress(f"C4: {e.src.size} edges, {nsteps} steps ({setup_s:.1f} s)")
    readers = []
    t0 = time.perf_counter()
    for k in range(nsteps):
        if k % 100 == 0:
            gstate.globals_ = {"tau": live_tau(gstate)}
        elif k % 100 == 1:
            gstate.globals_ = {"tau": np.float32(0.0)}
        gstate = step(gstate, px.StepInputs(xs_d[k], ys_d[k])).state
        readers.append(gstate._flag_reader("grown"))
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    grown = sum(int(r()) for r in readers)
    live = int(sum(int((b["dead"] == 0).sum().item()) for b in gstate.conns))
    progress(f"C4: {nsteps} steps in {elapsed:.2f} s, {grown} edges regrown, {live} live at the end")
    cpu = parity = None
    if not args.no_cpu_baseline:
        from oracle import oracle as ox
        from plastax_amd._plan import compile_plan

        ox.load()
        o = ox.OracleNet(static, host_units, host_conns, compile_plan(net, static), {"tau": np.float32(0.0)})
        o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
        pstate = fresh()
        pstep = px.make_step(net, static)
        times, same = [], True
        for k in range(2):
            tau = live_tau(pstate) if k == 0 else np.float32(0.0)
            pstate.globals_ = {"tau": tau}
            o.globals_ = {"tau": tau}
            res = pstep(pstate, px.StepInputs(xs_d[k], ys_d[k]))
            pstate = res.state
            t1 = time.perf_counter()
            lo = o.step(xs[k, 0], ys[k, 0])
            times.append(time.perf_counter() - t1)
            got = (int(pstate.grown), bool(pstate.overflow), bool(pstate.needs_resort), int(pstate.tail_start))
            same &= got == (o.grown, o.overflow, o.needs_resort, o.tail_start)
            same &= bool(np.float32(float(res.loss)).view(np.uint32) == np.float32(lo).view(np.uint32))
        units_ok = all(np.array_equal(column_to_numpy(pstate.units[n], uspecs[n]).view(np.uint8),
                                      o.units[n].view(np.uint8)) for n in uspecs)
        conns_ok = all(np.array_equal(column_to_numpy(b[n], cspecs[n]).view(np.uint8), o.conns[i][n].view(np.uint8))
                       for i, b in enumerate(pstate.conns) for n in cspecs)
        parity = {"steps": 2, "event_step_included": True, "flags_and_loss_equal": bool(same),
                  "units_bit_exact": bool(units_ok), "conns_bit_exact": bool(conns_ok)}
        progress(f"C4 parity over 2 steps: flags and loss {same}, units {units_ok}, conns {conns_ok}")
        sec = float(sum(times)) / 2
        cpu = {"value": 1.0 / sec, "unit": "steps/s", "cores": 1, "kind": "port",
               "sample": f"the first 2 steps of the same workload (a prune + regrow step and a plain one), "
                         f"{sec:.2f} s per step on average, the C oracle and oracle/growth.py, one thread"}
    ms = elapsed * 1e3 / nsteps
    line = {
        "metric": C4_METRIC,
        "value": round(1e3 / ms, 2),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": nsteps,
        "warmup": 0,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "C4: C3's 784-4096-4096-10 sparse MLP (10 % keep) at batch 1, tanh, softmax CE, "
                               "Adam(1e-3); every 100 steps PruneConn |w| < 10th percentile and ScoreAddConn "
                               "(32 x 32 shortlist per level, up to 1,024 new per level)",
                   "edges_start": int(e.src.size), "live_edges_end": live, "regrown_total": grown,
                   "events": (nsteps + 99) // 100},
        "roofline": None,
        "cpu_baseline": cpu,
        "full_size_parity": parity,
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(line), flush=True)
    return 0


C3_METRIC = "samples/sec per batched step (fwd+bwd+update, B=256) of C3's 784-4096-4096-10 sparse MLP"


def build_c3(px):
    grad = px.FieldSpec.float32("grad_pre_act")
    lossg = px.FieldSpec.float32("loss_grad")
    import plastax_amd.numpy as jnp

    class ReluForward(px.ForwardPass):
        combine = px.monoid.sum_

        def map(self, u, dst, src, c, cid, g):
            return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((px.ACTIVATION, jnp.maximum(acc, jnp.float32(0.0))))

    class ReluBackward(px.BackwardPass):
        combine = px.monoid.sum_

        def map(self, u, src, dst, c, cid, g):
            return c[px.WEIGHT, cid] * u[grad, dst]

        def apply(self, u, i, g, acc):
            gate = jnp.where(u[px.ACTIVATION, i] > 0, jnp.float32(1.0), jnp.float32(0.0))
            return px.UnitWrite.of((grad, (acc + u[lossg, i]) * gate))

    opt = px.optim.adam(1e-3, grad)

    class C3Net(px.Network):
        forward_pass = ReluForward()
        backward_pass = ReluBackward()
        loss = px.SoftmaxCrossEntropyLoss(lossg)
        update_conn = opt.update_conn()
        extra_unit_fields = (grad, lossg)
        extra_conn_fields = tuple(opt.state_fields)
        batch_reduction = px.MeanFloatFirstRest()

    return C3Net


def run_c2_prune(args) -> int:
    """C2 with a PruneConn every step under the three engines: "auto" (the
    predicate pass at the forward's slot), "triton" (the predicate inside the
    forward's edge pass) and "off" (the predicate pass at the prune slot):
    same steps, same kills; the losses and DEAD columns must agree."""
    import torch

    import plastax_amd as px
    import plastax_amd.numpy as jnp
    from plastax_amd import synth

    class HashPrune(px.PruneConn):
        """About one edge in 2^20 per step, from its ids and the step."""

        def predicate(self, u, c, cid, g):
            h = c[px.FROM_ID, cid] * jnp.int32(7) + c[px.TO_ID, cid] * jnp.int32(13) + g["step"]
            return (h % jnp.int32(1048573)) == jnp.int32(0)

    net0, e = build_c2(px, args.seed, args.scale)

    class C2Prune(net0):
        prune_conn = HashPrune()

    width = e.input_ids.size
    sign, perm = synth.c2_target(args.seed, width)
    nsteps = args.warmup + args.steps
    rng = np.random.default_rng(args.seed + 2)
    xs = rng.standard_normal((nsteps, width)).astype(np.float32)
    ts = np.ascontiguousarray((sign[None, :] * xs[:, perm]).astype(np.float32))
    dev = torch.device("cuda", 0)
    xs_d, ts_d = torch.from_numpy(xs).to(dev), torch.from_numpy(ts).to(dev)
    res = {}
    for mode in ("auto", "triton", "off"):
        static, state = px.NetworkBuilder.from_edges(
            C2Prune, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
            output_ids=e.output_ids, globals_={"step": np.int32(0)}, capacity_align=256, device="cpu")
        gstate = px.NetworkState({k: v.to(dev) for k, v in state.units.items()},
                                 tuple({k: v.to(dev) for k, v in b.items()} for b in state.conns),
                                 {"step": np.int32(0)})
        del state
        dead0 = sum(int(b["dead"].to(torch.int64).sum()) for b in gstate.conns)
        step = px.make_step(C2Prune, static, fuse_prune=mode)
        step.arena(gstate)
        losses = []
        for k in range(args.warmup):
            gstate.globals_ = {"step": np.int32(k)}
            r = step(gstate, px.StepInputs(xs_d[k], ts_d[k]))
            gstate = r.state
            losses.append(r.loss)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for k in range(args.warmup, nsteps):
            gstate.globals_ = {"step": np.int32(k)}
            r = step(gstate, px.StepInputs(xs_d[k], ts_d[k]))
            gstate = r.state
            losses.append(r.loss)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / args.steps
        dead = torch.cat([b["dead"].to(torch.int64) for b in gstate.conns])
        res[mode] = {"ms_per_step": ms, "fused": bool(step.prune_fusion.plan.fused),
                     "losses": torch.stack(losses).cpu().numpy(), "killed": int(dead.sum()) - dead0,
                     "dead": dead.cpu()}
        progress(f"C2 + PruneConn, fuse_prune={mode}: {ms:.4f} ms per step (fused: {res[mode]['fused']})")
        del gstate, step
        torch.cuda.empty_cache()
    same_loss = all(np.array_equal(res[m]["losses"].view(np.uint32), res["off"]["losses"].view(np.uint32))
                    for m in ("auto", "triton"))
    same_dead = all(torch.equal(res[m]["dead"], res["off"]["dead"]) for m in ("auto", "triton"))
    edges = int(e.src.size)
    line = {
        "metric": "ms per C2 streaming step with a PruneConn every step (fuse_prune='auto')",
        "value": round(res["auto"]["ms_per_step"], 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["auto"]["ms_per_step"], 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "C2 + PruneConn (edge-id hash, ~1 in 2^20 per step), Adam", "edges": edges,
                   "fused_single_pass_ms_per_step": round(res["triton"]["ms_per_step"], 4),
                   "prune_slot_pass_ms_per_step": round(res["off"]["ms_per_step"], 4)},
        "parity": {"losses_bit_exact": same_loss, "dead_equal": same_dead, "killed": res["triton"]["killed"]},
    }
    print(json.dumps(line), flush=True)
    return 0


def run_c1(args) -> int:
    """C1: the streaming PIPELINE net (1,024 units, 16,384 edges, SGD) run in
    chunks by Driver.scan: as captured HIP graphs (each chunk's first step
    eager, the rest one replay) and step by step, same chunks."""
    import torch

    import plastax_amd as px
    import plastax_amd.numpy as jnp
    from plastax_amd import synth
    from plastax_amd.driver import Driver
    from plastax_amd.state import column_to_numpy

    grad = px.FieldSpec.float32("grad_pre_act")
    lossg = px.FieldSpec.float32("loss_grad")

    class TanhForward(px.ForwardPass):
        combine = px.monoid.sum_

        def map(self, u, dst, src, c, cid, g):
            return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)))

    class TanhBackward(px.BackwardPass):
        combine = px.monoid.sum_

        def map(self, u, src, dst, c, cid, g):
            return c[px.WEIGHT, cid] * u[grad, dst]

        def apply(self, u, i, g, acc):
            a = u[px.ACTIVATION, i]
            return px.UnitWrite.of((grad, (acc + u[lossg, i]) * (jnp.float32(1.0) - a * a)))

    class MSELoss(px.Loss):
        seed_field = lossg

        def calculate_loss(self, u, outputs, targets, g):
            d = u.gather(px.ACTIVATION, outputs) - targets
            return jnp.sum(jnp.float32(0.5) * d * d), d

    opt = px.optim.sgd(1e-2, grad)

    class C1Net(px.Network):
        forward_pass = TanhForward()
        backward_pass = TanhBackward()
        loss = MSELoss()
        update_conn = opt.update_conn()
        extra_unit_fields = (grad, lossg)
        extra_conn_fields = opt.state_fields
        propagation = px.Propagation.PIPELINE

    e = synth.c1_pipeline(args.seed)
    a = synth.c1_target(args.seed)
    K = args.chunk
    nchunks = max(1, args.steps // K)
    rng = np.random.default_rng(args.seed + 7)
    xs = rng.standard_normal(((nchunks + 1) * K, e.input_ids.size)).astype(np.float32)
    ts = (xs @ a.T).astype(np.float32)
    dev = torch.device("cuda", 0)
    xs_d, ts_d = torch.from_numpy(xs).to(dev), torch.from_numpy(ts).to(dev)
    rates, first_records = {}, {}
    host = None
    for mode in ("graph", "step_by_step"):
        static, state = px.NetworkBuilder.from_edges(
            C1Net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
            output_ids=e.output_ids, globals_=None, device="cpu")
        if host is None:
            specs = {s.name: s for s in static.conn_fields}
            host = ({s.name: column_to_numpy(state.units[s.name], s).copy() for s in static.unit_fields},
                    [{n: column_to_numpy(b[n], specs[n]).copy() for n in specs} for b in state.conns], static)
        gstate = px.NetworkState({k: v.to(dev) for k, v in state.units.items()},
                                 tuple({k: v.to(dev) for k, v in b.items()} for b in state.conns), None)
        drv = Driver(C1Net, static, gstate)
        use_graph = mode == "graph"
        # warm-up chunk (captures the graph)
        first_records[mode] = drv.scan(px.StepInputs(xs_d[:K], ts_d[:K]), graph=use_graph).cpu().numpy()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for c in range(1, nchunks + 1):
            drv.scan(px.StepInputs(xs_d[c * K : (c + 1) * K], ts_d[c * K : (c + 1) * K]), graph=use_graph)
        torch.cuda.synchronize()
        rates[mode] = nchunks * K / (time.perf_counter() - t0)
        progress(f"C1 {mode}: {rates[mode]:.0f} steps/s")
    cpu = parity = None
    if not args.no_cpu_baseline:
        from oracle import oracle as ox
        from plastax_amd._plan import compile_plan

        ox.load()
        units, conns, static = host
        o = ox.OracleNet(static, {k: v.copy() for k, v in units.items()}, [{k: v.copy() for k, v in b.items()}
                                                                            for b in conns],
                         compile_plan(C1Net, static), None)
        t1 = time.perf_counter()
        ref = np.asarray([o.step(xs[i], ts[i]) for i in range(K)], dtype=np.float32)
        sec = time.perf_counter() - t1
        parity = {"steps": K, "graph_records_bit_exact": bool(np.array_equal(
            first_records["graph"].astype(np.float32).view(np.uint32), ref.view(np.uint32))),
                  "step_by_step_records_bit_exact": bool(np.array_equal(
            first_records["step_by_step"].astype(np.float32).view(np.uint32), ref.view(np.uint32)))}
        cpu = {"value": float(K / sec), "unit": "steps/s", "cores": 1, "kind": "port",
               "sample": f"{K} steps of the same workload, the C oracle (oracle/plastax_oracle.c), one thread"}
        progress(f"C1 parity over the first chunk: {parity}")
    line = {
        "metric": "steps/sec of C1's streaming pipeline net, Driver.scan in chunks (captured HIP graph)",
        "value": round(rates["graph"], 1),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": nchunks * K,
        "warmup": K,
        "ms_per_step": round(1e3 / rates["graph"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "C1: 1,024 tanh units, 16,384 edges, PIPELINE, MSE to a linear target, SGD(1e-2)",
                   "chunk": K, "step_by_step_steps_per_s": round(rates["step_by_step"], 1)},
        "cpu_baseline": cpu,
        "full_size_parity": parity,
    }
    print(json.dumps(line), flush=True)
    return 0


def measure_roofs(torch) -> dict:
    """The LDS and L2 read bandwidths of this GPU, measured live by the
    library's roof probes (plx_roof_probe: conflict-free 16-byte LDS reads;
    16-byte coalesced reads of a 2 MB L2-resident buffer), best of three."""
    import ctypes

    from plastax_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    out = torch.empty(2048 * 256, dtype=torch.int32, device=dev)
    buf = torch.ones(2 << 20, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    res = {}
    for name, kind, iters in (("lds", _lib.PLX_PROBE_LDS, 2000), ("l2", _lib.PLX_PROBE_L2, 200)):
        best = 0.0
        for _ in range(3):
            nbytes, ms = ctypes.c_double(), ctypes.c_float()
            _lib.check(lib.plx_roof_probe(kind, iters, buf.data_ptr(), buf.numel(), out.data_ptr(),
                                          ctypes.byref(nbytes), ctypes.byref(ms), stream), "plx_roof_probe")
            best = max(best, nbytes.value / (ms.value * 1e-3) / 1e9)
        res[name + "_read_gbs"] = round(best, 1)
    return res


def run_c3(args) -> int:
    """C3: the batched step (B = 256) of the 784-4096-4096-10 sparse MLP."""
    import torch

    import plastax_amd as px
    from plastax_amd import synth
    from plastax_amd.state import column_to_numpy

    B = 256
    t_setup = time.perf_counter()
    net = build_c3(px)
    e = synth.c3_mlp(args.seed)
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, device="cpu")
    specs = {s.name: s for s in static.conn_fields}
    host_units = {s.name: column_to_numpy(state.units[s.name], s).copy() for s in static.unit_fields}
    host_conns = [{n: column_to_numpy(b[n], specs[n]).copy() for n in specs} for b in state.conns]
    dev = torch.device("cuda", 0)
    gstate = px.NetworkState(
        {k: v.to(dev) for k, v in state.units.items()},
        tuple({k: v.to(dev) for k, v in b.items()} for b in state.conns),
        None,
    )
    step = px.make_step(net, static, batch_size=B)
    nsteps = args.warmup + args.steps
    xs, ys = synth.c3_batches(args.seed, nsteps, B)
    xs_d, ys_d = torch.from_numpy(xs).to(dev), torch.from_numpy(ys).to(dev)
    step.arena(gstate)
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup
    progress(f"C3: {e.src.size} edges, B = {B} ({setup_s:.1f} s)")
    first_loss = None
    first_units = first_conns = None
    for k in range(args.warmup):
        res = step(gstate, px.StepInputs(xs_d[k], ys_d[k]))
        gstate = res.state
        if k == 0:
            first_loss = res.loss
            if not args.no_cpu_baseline:
                # every column after the first step, for the full-size parity check
                first_units = {s.name: column_to_numpy(gstate.units[s.name], s).copy() for s in static.unit_fields}
                first_conns = [{n: column_to_numpy(b[n], specs[n]).copy() for n in specs} for b in gstate.conns]
    torch.cuda.synchronize()
    dominant = "update_conn"
    timer = EventTimer({dominant})
    step.timer = timer
    timer.on = True
    t0 = time.perf_counter()
    last = None
    for k in range(args.warmup, nsteps):
        last = step(gstate, px.StepInputs(xs_d[k], ys_d[k]))
        gstate = last.state
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    timer.on = False
    dom = timer.summary()[dominant]
    breakdown = EventTimer()
    step.timer = breakdown
    breakdown.on = True
    for k in range(min(3, nsteps)):
        gstate = step(gstate, px.StepInputs(xs_d[k], ys_d[k])).state
    breakdown.on = False
    step.timer = None
    kernels = breakdown.summary()
    kernels = kernel_table(kernels)
    edges = int(e.src.size)
    ms = elapsed * 1e3 / args.steps
    # The tiled batch-mean update (plx_update_batch_tiles) reads, per live
    # edge, its position (4 B) and packed tile-local ids (2 B), WEIGHT and the
    # optimizer state it keeps per edge, and writes WEIGHT and that state
    # back: Adam with the step count uniform over the bucket keeps m and v
    # (t is one number), so 4 + 2 + 12 read + 12 written = 30 B; DEAD is read
    # only when tombstones sit inside the live range. It also gathers two
    # B-wide unit rows per tile (L2-served, counted apart).
    # Its bound is LDS, not HBM: every edge reads both staged B-wide rows,
    # g[dst, b] and act[src, b], from LDS for every sample (8 B per edge and
    # sample; rocprofv3's SQ_INSTS_LDS_LOAD_BANDWIDTH counts the same bytes),
    # against 30 B per edge of HBM. The roof is this GPU's LDS read
    # bandwidth, measured live by the library's probe.
    arena = gstate._arena
    uniform_t = all(t is not None for t in arena.t_now)
    state_cols = 2 if uniform_t else 3
    per_edge = 4 + 2 + 4 * (1 + state_cols) * 2 + (1 if arena.dead_in_rows else 0)
    per_launch_hbm = per_edge * edges * args.steps / dom["launches"]
    per_launch_lds = 8 * B * edges * args.steps / dom["launches"]
    secs = dom["mean_ms"] * 1e-3
    roofs = measure_roofs(torch)
    ach_lds = per_launch_lds / secs / 1e9
    ach_hbm = per_launch_hbm / secs / 1e9
    roofline = {
        "kernel": "update_conn (plx_update_batch_tiles)",
        "bound": "lds",
        "achieved": round(ach_lds, 1),
        "peak": roofs["lds_read_gbs"],
        "unit": "GB/s",
        "frac": round(ach_lds / roofs["lds_read_gbs"], 4),
        "traffic": None,
        "peak_source": "measured live: plx_roof_probe, conflict-free 16-byte LDS reads on every CU",
        "lds_bytes_per_edge_sample": 8,
        "algorithmic_lds_bytes_per_launch": int(per_launch_lds),
        "mean_launch_ms": round(dom["mean_ms"], 4),
        "hbm": {"bytes_per_edge": per_edge, "algorithmic_bytes_per_launch": int(per_launch_hbm),
                "achieved": round(ach_hbm, 1), "peak": HBM_PEAK_GBS, "frac": round(ach_hbm / HBM_PEAK_GBS, 4)},
        "l2_read_peak_gbs": roofs["l2_read_gbs"],
    }
    cpu = None
    parity = None
    if not args.no_cpu_baseline:
        from oracle import batched as ob
        from oracle import oracle as ox
        from plastax_amd._plan import compile_plan

        ox.load()
        o = ox.OracleNet(static, host_units, host_conns, compile_plan(net, static), None)
        orc = ob.OracleBatch(o, B)
        t1 = time.perf_counter()
        ref_loss = np.float32(orc.step(xs[0], ys[0]))
        sec = time.perf_counter() - t1
        if first_loss is not None:
            # Full-size parity: the first batched step's loss and every unit
            # and connection column after it, bit for bit.
            got = np.float32(float(first_loss))

            def same(a, b):  # bitwise for float32 (NaN == NaN, -0.0 != +0.0), by value otherwise
                a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
                if a.dtype == np.float32:
                    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))
                return bool(np.array_equal(a, b))

            units_ok = all(same(first_units[n], o.units[n]) for n in first_units)
            conns_ok = all(same(c[n], oc[n]) for c, oc in zip(first_conns, o.conns) for n in c)
            parity = {"steps": 1, "loss_bit_exact": bool(got.view(np.uint32) == ref_loss.view(np.uint32)),
                      "units_bit_exact": bool(units_ok), "conns_bit_exact": bool(conns_ok)}
            progress(f"C3 parity after step 1: loss {parity['loss_bit_exact']}, units {units_ok}, conns {conns_ok}")
        cpu = {
            "value": float(B / sec),
            "unit": "samples/s",
            "cores": 1,
            "kind": "port",
            "sample": f"1 batched step of the same workload (B = 256), {sec:.1f} s, the C oracle per sample "
            "plus numpy batch reductions (oracle/batched.py), one thread",
        }
    line = {
        "metric": C3_METRIC,
        "value": round(B / (ms * 1e-3), 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "C3: 784-4096-4096-10 sparse MLP (10 % keep), ReLU, softmax CE, Adam(1e-3), B = 256",
            "edges": edges,
            "batch": B,
            "edge_samples_per_s": round(edges * B / (ms * 1e-3), 1),
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "full_size_parity": parity,
        "kernels": kernels,
        "loss_last": float(last.loss),
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", choices=("c1", "c2", "c2_prune", "c3", "c4", "c5", "c5_growth"), default="c2",
                    help="c1: the small streaming PIPELINE net run by Driver.scan (graph vs step by step); "
                    "c2: the streaming step (the headline metric); c3: the batched step (B = 256); "
                    "c5: the growing reservoir end to end; c5_growth: its add_conn phase alone")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help=f"timed steps (default: {C2_DEFAULT_STEPS} for c2, about five seconds of GPU work; "
                    "200 for the other workloads)")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--scale", type=int, default=1, help="shrink C2's layer width (tests only)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-steps", type=int, default=12)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--chunk", type=int, default=100, help="c1: steps per Driver.scan chunk")
    ap.add_argument("--c4-steps", type=int, default=5000, help="c4: steps of the run (events every 100)")
    ap.add_argument("--relayout", choices=("merge", "full"), default="merge",
                    help="c5: the churn layout after a growth step: merged from the previous one, or built again")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain elementwise copy of MIB MiB (read MIB, write MIB) "
                    "five times: the reference kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = C2_DEFAULT_STEPS if args.workload == "c2" else 200
    if args.gpus != 1:
        print(
            f"bench.py: --gpus {args.gpus} is not supported: this build measures the step on one "
            "GPU (the single-GPU kernel runs on the full arena); multi-GPU sharding is out of scope",
            file=sys.stderr,
        )
        return 2

    import torch

    if args.workload == "c5_growth":
        return run_c5_growth(args)
    if args.workload == "c1":
        return run_c1(args)
    if args.workload == "c2_prune":
        return run_c2_prune(args)
    if args.workload == "c3":
        return run_c3(args)
    if args.workload == "c4":
        return run_c4(args)
    if args.workload == "c5":
        return run_c5(args)

    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.randn(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        progress(f"copy calibration: 5 x {args.copy_calibration} MiB read + write")
        return 0

    import plastax_amd as px
    from plastax_amd.state import column_to_numpy

    t_setup = time.perf_counter()
    net, e = build_c2(px, args.seed, args.scale)
    progress(f"synthetic C2 edges: {e.src.size} ({time.perf_counter() - t_setup:.1f} s)")
    from plastax_amd import synth

    width = e.input_ids.size
    static, state = px.NetworkBuilder.from_edges(
        net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
        output_ids=e.output_ids, globals_=None, capacity_align=256, device="cpu")
    progress(f"logical arena built ({time.perf_counter() - t_setup:.1f} s)")
    specs = {s.name: s for s in static.conn_fields}
    host_units = {s.name: column_to_numpy(state.units[s.name], s).copy() for s in static.unit_fields}
    host_conns = [{n: column_to_numpy(b[n], specs[n]).copy() for n in specs} for b in state.conns]
    dev = torch.device("cuda", 0)
    gstate = px.NetworkState(
        {k: v.to(dev) for k, v in state.units.items()},
        tuple({k: v.to(dev) for k, v in b.items()} for b in state.conns),
        None,
    )
    del state
    step = px.make_step(net, static)
    sign, perm = synth.c2_target(args.seed, width)
    nsteps = args.warmup + args.steps
    rng = np.random.default_rng(args.seed + 2)
    # Step k streams sample k % pool of a pool of synthetic samples (a long
    # run needs no more host or device memory for its inputs).
    pool = min(nsteps, C2_INPUT_POOL)
    xs = rng.standard_normal((pool, width)).astype(np.float32)
    # (dense rows: numpy's fancy indexing returns a column-major array)
    ts = np.ascontiguousarray((sign[None, :] * xs[:, perm]).astype(np.float32))
    xs_d = torch.from_numpy(xs).to(dev)
    ts_d = torch.from_numpy(ts).to(dev)
    step.arena(gstate)  # physical layout build (host, once)
    progress(f"physical arena on the device ({time.perf_counter() - t_setup:.1f} s)")
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup

    # The losses of the first steps (warm-up and timed) are kept, on the
    # device, for the full-size parity check against the CPU oracle's steps.
    dev_losses = []
    for k in range(args.warmup):
        res = step(gstate, px.StepInputs(xs_d[k % pool], ts_d[k % pool]))
        gstate = res.state
        if k <= args.cpu_steps:
            dev_losses.append(res.loss)
    torch.cuda.synchronize()

    # The timed region records HIP events around the dominant kernel (the
    # fused backward + update) only, one launch in per_step + 1, so that the
    # sampled launches rotate over the buckets (a step launches it for
    # buckets nb-1 .. 1, in that order); a short pass afterwards times every
    # launch kind for the breakdown.
    dominant = "backward_update"
    arena = gstate._arena
    per_step = arena.num_buckets - 1
    timer = EventTimer({dominant}, stride=per_step + 1)
    step.timer = timer
    timer.on = True
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    last = None
    for k in range(args.warmup, nsteps):
        last = step(gstate, px.StepInputs(xs_d[k % pool], ts_d[k % pool]))
        gstate = last.state
        if k <= args.cpu_steps:
            dev_losses.append(last.loss)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    timer.on = False
    dom = timer.summary()[dominant]
    loss = float(last.loss)
    breakdown = EventTimer()
    step.timer = breakdown
    breakdown.on = True
    for k in range(min(5, nsteps)):
        gstate = step(gstate, px.StepInputs(xs_d[k], ts_d[k])).state
    breakdown.on = False
    step.timer = None
    kernels = breakdown.summary()

    edges = int(e.src.size)
    n_units = int(e.num_units)
    ms_per_step = elapsed * 1e3 / args.steps
    value = edges / (elapsed / args.steps)
    step_bytes = 54 * edges + 16 * n_units
    step_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9

    # Algorithmic bytes per step of each launch kind (the reference column
    # model): the forward reads FROM_ID, TO_ID, DEAD, WEIGHT (13 B/edge) of
    # every bucket; the fused backward+update and the update-only pass read
    # FROM_ID, TO_ID, DEAD, WEIGHT, m, v, t and write WEIGHT, m, v, t
    # (41 B/edge), the former over buckets 1.., the latter over bucket 0.
    lives = [int(v) for v in arena.lives]
    bytes_per_step = {
        "forward": 13 * sum(lives),
        "backward_update": 41 * sum(lives[1:]),
        "update_conn": 41 * lives[0],
    }
    roofline = None
    if dominant in bytes_per_step:
        # The sampled launches' own buckets: ordinal c is bucket nb-1 - c % per_step.
        sampled = [41 * lives[arena.num_buckets - 1 - c % per_step] for c in dom["ordinals"]]
        per_launch = float(np.mean(sampled))
        ach = sum(sampled) / (dom["total_ms"] * 1e-3) / 1e9
        roofline = {
            "kernel": dominant,
            "bound": "hbm",
            "achieved": round(ach, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4),
            "traffic": None,
            "algorithmic_bytes_per_launch": int(per_launch),
            "mean_launch_ms": round(dom["mean_ms"], 4),
            "sampled_launches": dom["launches"],
        }
    # HBM traffic per launch is a profile figure (rocprofv3 FETCH_SIZE and
    # WRITE_SIZE of the dominant kernel, scaled by a plain copy), measured at
    # the commit the file names, not in this run.
    traffic_file = ROOT / "profiles" / "traffic.json"
    if roofline is not None and traffic_file.exists():
        tf = json.loads(traffic_file.read_text())
        roofline["traffic"] = tf.get(dominant)
        roofline["traffic_source"] = {k: tf.get(k) for k in ("measured_at", "kernel", "method") if k in tf}

    cpu = None
    parity = None
    progress(f"timed {args.steps} steps: {elapsed * 1e3 / args.steps:.3f} ms/step")
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(px, net, static, e, host_units, host_conns, xs, ts, args.cpu_steps)
        # Full-size parity: the device's loss of each of the first steps, bit
        # for bit against the oracle's on the same inputs (the loss of step k
        # reads every weight after k updates).
        refs = cpu.pop("losses")
        got = [np.float32(float(x)) for x in dev_losses]
        parity = {}
        for leg, ref in refs.items():
            m = min(len(ref), len(got))
            same = [bool(np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32))
                    for a, b in zip(got[:m], ref[:m])]
            parity[leg] = {"steps": m, "loss_bit_exact": all(same),
                           "first_mismatch": None if all(same) else same.index(False)}
            progress(f"full-size parity over {m} steps vs the {leg} oracle: "
                     f"{'bit-exact' if all(same) else 'MISMATCH'}")
        parity = {"steps": min(p["steps"] for p in parity.values()),
                  "loss_bit_exact": all(p["loss_bit_exact"] for p in parity.values()), "legs": parity}

    kernels = kernel_table(kernels)
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "edges/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "C2: 8x131072 tanh units, 2^26 Zipf(1.1) edges, MSE, Adam, batch 1 streaming",
            "edges": edges,
            "units": n_units,
            "layers": 8,
            "optimizer": "adam(1e-3)",
            "scale": args.scale,
            "input_pool": pool,
        },
        "step_hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        "step_algorithmic_gbs": round(step_gbs, 1),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "full_size_parity": parity,
        "kernels": kernels,
        "loss_last": loss,
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
