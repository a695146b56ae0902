"""``make_step``: assemble a network's phases into one device step.

Mirrors src/plastax/step.py:76-237 and :545-626. ``make_step(net, static)``
traces the net's policies once (plastax_amd._plan) and returns a callable
``step(state, inputs) -> StepResult``. A call runs, on torch's current HIP
stream and without a host synchronisation: the input scatter (step.py:598),
the forward level walk, the loss, the backward level walk and the fused
connection update (phases.py:150-157), then bumps ``state.step``. The state
is donated (step.py:624): its buffers are updated in place and the returned
``StepResult.state`` owns them.
"""

from __future__ import annotations

import dataclasses
from typing import Any, Literal

import numpy as np
import torch

from plastax_amd import _lib
from plastax_amd._expr import UnsupportedPolicyError
from plastax_amd._layout import NSUPER, TILE, Arena
from plastax_amd._plan import Plan, compile_plan, program_struct
from plastax_amd._types import ACTIVATION, DEAD, Propagation
from plastax_amd.fusion import PruneFusionPlan, PruneFusionRecord, plan_prune_fusion
from plastax_amd.state import NetworkState, NetworkStatic

# The fused forward + PruneConn sweep ("hip" engine): "compiled" runs the
# predicate compiled into the forward kernel (plx_forward_prune_compile);
# "interpreted" evaluates it with the site interpreter inside the library's
# forward kernel (tests). Both give the same bits.
FUSED_PREDICATE: str = "compiled"


@dataclasses.dataclass(frozen=True)
class StepInputs:
    """Clamped inputs and loss targets of one step (phases.py:72-84)."""

    inputs: Any
    targets: Any = None


class StepResult:
    """A step's output (step.py:45-67): the new state, the growth overflow
    flag, the loss (a 0-d float32 device tensor) and the dropped growth
    candidates (None without growth). ``overflow`` may be given as a
    zero-argument callable: it is then read (from the device) on first
    access, so returning the result waits for nothing."""

    __slots__ = ("state", "loss", "growth_remainder", "_overflow")

    def __init__(self, state: NetworkState, overflow: Any, loss: Any, growth_remainder: Any = None) -> None:
        self.state = state
        self.loss = loss
        self.growth_remainder = growth_remainder
        self._overflow = overflow

    @property
    def overflow(self) -> Any:
        if callable(self._overflow):
            self._overflow = self._overflow()
        return self._overflow

    def __repr__(self) -> str:
        return f"StepResult(state={self.state!r}, loss={self.loss!r})"


def make_step(
    net: type,
    static: NetworkStatic,
    *,
    batch_size: int | None = None,
    layout: Literal["auto", "edge_list", "csr", "triton"] = "auto",
    fuse_prune: Literal["auto", "triton", "xla", "off"] = "auto",
    growth: Literal["auto", "xla", "triton"] = "auto",
) -> "StepFn":
    """Build the device step of ``net`` (step.py:76-237).

    Raises ValueError on the reference's argument errors and
    UnsupportedPolicyError for a policy the device path cannot run.
    """
    if batch_size is not None:
        if batch_size < 1:
            raise ValueError(f"make_step: batch_size must be >= 1, got {batch_size}")
        if net.propagation is Propagation.PIPELINE:
            raise ValueError(
                "make_step: batch_size is for TOPOLOGICAL (feed-forward) nets; a "
                "PIPELINE net carries per-sample recurrent state between steps"
            )
        if net.batch_reduction is None:
            raise ValueError(
                f"make_step: a batched step needs {net.__name__}.batch_reduction"
            )
    if layout not in ("auto", "edge_list", "csr", "triton"):
        raise ValueError(f"make_step: unknown layout {layout!r}")
    if fuse_prune not in ("auto", "triton", "xla", "off"):
        raise ValueError(f"make_step: unknown fuse_prune {fuse_prune!r}")
    if growth not in ("auto", "xla", "triton"):
        raise ValueError(f"make_step: unknown growth engine {growth!r}")
    if batch_size is not None:
        from plastax_amd.batched import BatchedStepFn

        step = BatchedStepFn(compile_plan(net, static), static, batch_size)
    else:
        step = StepFn(compile_plan(net, static), static)
    step.prune_fusion = PruneFusionRecord(fuse_prune)
    return step


def _stream(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


class StepFn:
    """The callable ``make_step`` returns."""

    def __init__(self, plan: Plan, static: NetworkStatic) -> None:
        self.plan = plan
        self.static = static
        self._dev_consts: dict[Any, Any] = {}
        # Optional hook with begin(kind) / end(kind), called around every
        # kernel launch on the launching stream (the benchmark records HIP
        # events there).
        self.timer: Any = None
        # Positions per backward tile, and superblocks per bucket at most, of
        # the arenas this step builds.
        self.tile: int = TILE
        self.nsuper: int = NSUPER
        # The arena layout: "tiled" (host-built tiles: the fast streaming
        # backward), "churn" (rebuilt on the device after every structural
        # change; the backward folds each source's edges in slot order), or
        # "auto": churn when growth fires every step.
        self.arena_mode: str = "auto"
        # Where the tiled layout is built: "device" (plastax_amd._layout_dev)
        # or "host" (plastax_amd._layout, numpy); the tables are equal.
        self.layout_build: str = "device"
        # How the churn layout follows a growth step: "merge" (the claimed
        # slots merged into the previous layout) or "full" (built again from
        # the logical buckets); the layouts are equal.
        self.relayout: str = "merge"
        # Unit and structural phases, traced on the first step (their
        # programs read the globals' structure).
        self._update_unit: Any = None
        self._update_generic: Any = None
        self._prune_unit: Any = None
        self._prune: Any = None
        self._add_unit: Any = None
        self._grow: Any = None
        # prune_conn inside the forward sweep (phases.py:1629-1848), planned
        # on the first call.
        self.prune_fusion = PruneFusionRecord("auto")

    def _launch(self, kind: str, fn: Any, *args: Any) -> None:
        timer = self.timer
        if timer is not None:
            timer.begin(kind)
        _lib.check(fn(*args), kind)
        if timer is not None:
            timer.end(kind)

    # -- per-device constants ------------------------------------------------
    def _consts(self, device: torch.device, arena: Arena) -> dict[str, Any]:
        """Device constants of a step on ``arena``: input / output ids and the
        input mask in the arena's unit order, and Adam's power table."""
        key = (device.type, device.index)
        if key not in self._dev_consts:
            c = {}
            if self.plan.update is not None and self.plan.update.rule_code == 2:
                c["pow_table"] = torch.from_numpy(self.plan.pow_table()).to(device)
            self._dev_consts[key] = c
        c = dict(self._dev_consts[key])
        c["input_ids"] = arena.input_ids
        c["output_ids"] = arena.output_ids
        c["is_input"] = arena.is_input
        c["unit_map"] = arena.uinv  # logical unit id -> its row in the laid-out columns (host)
        return c

    def churn(self) -> bool:
        """Whether this step lays its arena out with the churn layout."""
        if self.arena_mode != "auto":
            if self.arena_mode not in ("tiled", "churn"):
                raise ValueError(f"arena_mode must be 'auto', 'tiled' or 'churn', got {self.arena_mode!r}")
            return self.arena_mode == "churn"
        if self.plan.backward is not None and self.plan.backward.generic is not None:
            return True  # a generic backward folds each source's out-edges from the churn lists
        cfg = self.plan.add_conn
        if cfg is None:
            return False
        every = cfg.trigger == "every_step" or (isinstance(cfg.trigger, tuple) and int(cfg.trigger[1]) == 1)
        return every and int(getattr(self.plan.net, "structural_interval", 1)) == 1

    @property
    def backward_order(self) -> str:
        """"slot": each source's terms in logical slot order (the churn
        layout); "tiled": the tiled layout's tile / superblock order."""
        return "slot" if self.churn() else "tiled"

    def arena(self, state: NetworkState) -> Arena:
        """The state's physical arena (built on first use)."""
        if state._arena is None:
            if self.churn():
                from plastax_amd._churn import ChurnArena

                prev, state._arena_prev = state._arena_prev, None
                if self.relayout not in ("merge", "full"):
                    raise ValueError(f"relayout must be 'merge' or 'full', got {self.relayout!r}")
                if prev is None or self.relayout == "full":
                    prev = (None, None, None)
                state._arena = ChurnArena(self.static, state.units, state._conns, state.device,
                                          _stream(state.device), prev=prev[0], dead_before=prev[1],
                                          claim_bound=prev[2])
            elif self.layout_build == "device":
                from plastax_amd._layout_dev import DeviceArena

                state._arena = DeviceArena(self.static, state.units, state._conns, state.device,
                                           _stream(state.device), tile=self.tile, nsuper=self.nsuper)
            elif self.layout_build == "host":
                state._arena = Arena(
                    self.static, state.units, state._conns, state.device, tile=self.tile,
                    nsuper=self.nsuper,
                )
            else:
                raise ValueError(f"layout_build must be 'device' or 'host', got {self.layout_build!r}")
            up = self.plan.update
            if up is not None and up.rule_code == 2:
                state._arena.init_uniform_t(up.state_columns()[2])
            state._arena_ahead = False
        return state._arena

    @staticmethod
    def _edge_state(d: Any, arena: Arena, b: int, update: bool) -> None:
        """Liveness and Adam step-count fields of a tile / update descriptor."""
        d.live_end = arena.live_end(b)
        d.dead = arena.cols["dead"].data_ptr() if arena.dead_in_rows else None
        if update and arena.t_now and arena.t_now[b] is not None:
            d.step_mode = 1
            d.step_t = arena.t_now[b]

    @staticmethod
    def _advance_t(arena: Arena, b: int) -> None:
        if arena.t_now and arena.t_now[b] is not None:
            arena.t_now[b] += 1.0

    # -- the step ------------------------------------------------------------
    def __call__(self, state: NetworkState, inputs: StepInputs) -> StepResult:
        plan = self.plan
        dev = state.device
        if dev.type != "cuda":
            raise RuntimeError("the plastax_amd step runs on a GPU; the state lives on the CPU")
        lib = _lib.load()
        state = state._donate()
        arena = self.arena(state)
        consts = self._consts(dev, arena)
        stream = _stream(dev)
        units = state._physical_units(arena)
        n_units = self.static.num_units

        # Input scatter (step.py:598).
        n_in = len(self.static.input_ids)
        if n_in:
            # (the kernels read dense arrays: a strided view is copied)
            x_in = torch.as_tensor(inputs.inputs, dtype=torch.float32, device=dev).reshape(-1).contiguous()
            if x_in.numel() != n_in:
                raise ValueError(f"step: expected {n_in} inputs, got {x_in.numel()}")
            _lib.check(
                lib.plx_scatter_f32(
                    n_in,
                    consts["input_ids"].data_ptr(),
                    x_in.data_ptr(),
                    units[ACTIVATION.name].data_ptr(),
                    stream,
                ),
                "plx_scatter_f32",
            )

        fin_common = dict(
            level=units["level"].data_ptr(),
            is_input=consts["is_input"].data_ptr(),
            pruned=units["pruned"].data_ptr() if "pruned" in units else None,
        )
        g = state.globals_

        # Forward (phases.py:942-1015).
        if plan.forward.generic is not None:
            self._forward_generic(arena, units, g, stream)
        else:
            fp = plan.forward
            swaps = self._shadow(units, fp.program.out_fields) if arena.pipeline else {}
            acc = None
            if arena.fwd_carry:
                acc = torch.empty(n_units, dtype=torch.float32, device=dev)
                _lib.call("plx_fill_f32", n_units, fp.identity, acc.data_ptr(), stream)
            prog = program_struct(fp.program, units, g, out_override=swaps)
            fusion = self._fusion_plan(g)
            fused = self._fused_prune_progs(arena, units, fin_common, g, stream) if fusion.fused else None
            for b in range(arena.num_buckets):
                rows = arena.fwd[b]
                d = _lib.plx_forward_desc()
                d.nrows = rows.nrows
                d.monoid = fp.monoid
                d.tbl_base, d.tbl_len = arena.src_table(b)
                d.row_unit = rows.rows.data_ptr()
                d.row_ptr = rows.ptr.data_ptr()
                d.src = arena.cols["from_id"].data_ptr()
                d.weight = arena.cols["weight"].data_ptr()
                # Row ranges hold live positions only unless tombstones were set
                # inside them after the layout was built.
                d.dead = arena.cols["dead"].data_ptr() if arena.dead_in_rows else None
                d.x = fp.gathered(units, ACTIVATION.name).data_ptr()
                d.map = fp.map_struct()
                d.acc = acc.data_ptr() if acc is not None else None
                d.fin.level = fin_common["level"]
                d.fin.is_input = fin_common["is_input"]
                d.fin.pruned = fin_common["pruned"]
                d.fin.fin_level = -1 if arena.pipeline else b + 1
                d.fin.skip_inputs = 1
                d.apply = prog
                handle = None
                if fused is not None and fusion.engine == "hip":
                    d.prune_prog = fused[b].data_ptr()
                    d.prune_sink = arena.prune_sink.data_ptr()
                    d.prune_slot = arena.slot[arena.bases[b]:].data_ptr()
                    d.ids_logical, d.ids_physical = arena.uperm32.data_ptr(), arena.uinv32.data_ptr()
                    d.prune_base = arena.bases[b]
                    d.num_units = n_units
                    handle = self._fused_handle
                if handle is not None:
                    self._launch("forward", lib.plx_forward_bucket_compiled, handle, d, stream)
                else:
                    self._launch("forward", lib.plx_forward_bucket, d, stream)
            self._unshadow(units, swaps)
            if fused is not None and fusion.engine == "xla":
                self._xla_prune(arena, g, stream)

        # Loss (phases.py:1107-1131).
        if plan.loss is not None:
            loss = torch.empty((), dtype=torch.float32, device=dev)
            self._loss(plan, units, inputs, consts, loss, stream, g)
        else:
            loss = torch.zeros((), dtype=torch.float32, device=dev)

        # Backward (phases.py:1018-1104) and connection update
        # (phases.py:1196-1242). In a TOPOLOGICAL step they share one pass per
        # bucket: no update_unit runs between them (the plan refuses one),
        # bucket b's backward terms use its pre-update weights, and bucket b's
        # update needs only finalized grads (levels > b) and activations.
        self._backward_update(plan, arena, units, consts, fin_common, stream, g)
        if plan.update is not None or plan.update_generic:
            state._mark_ahead()

        # Structural phases (phases.py:1245-1498, :4490-5203).
        if plan.prune_unit or plan.prune_conn or plan.add_unit or plan.add_conn is not None:
            self._structural(state, arena, units, stream, g)
        # reset_global (phases.py:87-182, last): the globals live on the host.
        if plan.reset_global:
            state.globals_ = plan.net.reset_global.reset(state.globals_)

        state.step = state.step + 1
        return StepResult(state=state, overflow=state._flag_reader("overflow"), loss=loss, growth_remainder=None)

    def _structural(self, state: NetworkState, arena: Arena, units: dict, stream: int, g: Any) -> None:
        """prune_unit and PruneConn on the physical arena (tombstones set in
        place), then add_unit and add_conn on the logical arena (the
        caller's unit ids; slot order). New units or a growth that fired
        replace the logical columns, and the next step lays the arena out
        again."""
        from plastax_amd import grow, units as unit_phases

        plan = self.plan
        k = grow.Kernels(state.device, stream)
        if plan.prune_unit:
            if self._prune_unit is None:
                self._prune_unit = unit_phases.PruneUnitPhase(plan.net, self.static, g)
            doomed, _ = self._prune_unit.run(k, units, g, site_ids=arena.uperm32, ids_physical=arena.uinv32)
            self._prune_unit.kill(k, arena, doomed)
            # Whether anything died stays on the device: from here on the
            # kernels read DEAD inside the live ranges.
            arena.dead_in_rows = True
            state._mark_ahead({DEAD.name, arena.t_name})  # tombstones and their stamped step counts
        if plan.prune_conn:
            if self._prune is None:
                self._prune = grow.PruneConnPhase(plan.net, self.static, g)
            timer = self.timer
            if timer is not None:
                timer.begin("prune_conn")
            if self.prune_fusion.plan is not None and self.prune_fusion.plan.fused:
                self._merge_prune(arena, stream)  # build_prune_merge_phase (phases.py:2447-2469)
            else:
                self._prune.run_physical(k, arena, units, g)
            if timer is not None:
                timer.end("prune_conn")
            arena.dead_in_rows = True
            state._mark_ahead({DEAD.name, arena.t_name})
        spawned = False  # add_unit ran: its flags stay on the device until read
        if plan.add_unit:
            if self._add_unit is None:
                self._add_unit = unit_phases.AddUnitPhase(plan.net, self.static, g)
            phase_u = self._add_unit
            if phase_u.fires(int(state.step)):
                before_units = state.units
                # The phase writes the new units into free slots of these
                # columns in place (the state was donated to the step, and
                # the spawned units read only their parents' values).
                ulog = dict(before_units)
                flags = phase_u.run_device(k, ulog, g)
                if self._grow is not None:
                    self._grow.carry_level_bound(before_units["level"], ulog["level"], phase_u.level_bound)
                state._defer_flag("units_added", flags, 0)
                state._defer_flag("unit_overflow", flags, 1)
                state.units = ulog
                spawned = True
            else:
                state.units_added, state.unit_overflow = 0, False

        def relayout_for_new_units() -> None:
            # New units need rows in the layout: the arena is laid out again
            # (a growth that fires replaces the buckets and does it anyway).
            if spawned and state.units_added:
                state.conns = state.conns

        if plan.add_conn is None:
            relayout_for_new_units()
        else:
            if self._grow is None:
                self._grow = grow.AddConnPhase(plan.net, self.static, g)
            phase = self._grow
            # (units_added is read only for a growth triggered by it)
            added = int(state.units_added) if phase.cfg.trigger == "on_units_added" else 0
            fires = phase.cfg.fires(phase.ac, step=int(state.step), interval=phase.interval,
                                    units_added=added, globals_=g)
            if not fires:
                state.grown, state.overflow = 0, False
                relayout_for_new_units()
                return
            conns = state.conns  # the logical view, in step with the arena
            prev = state._arena
            before: Any = None
            listed = False
            if getattr(prev, "churn", False):
                if phase.claims_listable(state.units["level"]):
                    # the claim lists the slots it fills (grow.ClaimedSlots)
                    listed = phase.want_claimed = True
                else:
                    # DEAD before the claim: the claimed slots are the ones it turns live
                    before = [bucket[DEAD.name].clone() for bucket in conns]
            phase.claimed = None
            # The flags stay on the device from step to step: the tail start
            # (PIPELINE) and needs_resort go in as the last claim's device
            # values, and this claim's flags are read only when the caller
            # asks (as the reference's Driver reads them after its step).
            tail_src = state._flag_source("tail_start")
            tail = tail_src[0][tail_src[1] : tail_src[1] + 1] if tail_src is not None else int(state.tail_start)
            resort_src = state._flag_source("needs_resort")
            out = phase.run(k, state.units, conns, step=int(state.step), globals_=g, tail_start=tail,
                            units_added=added,
                            needs_resort=resort_src if resort_src is not None else bool(state.needs_resort))
            phase.want_claimed = False
            state.conns = out.conns
            if listed:
                before = phase.claimed  # (None: not listed; the next layout is built afresh)
            if before is not None:
                # the next layout merges the claimed slots into prev's, sized
                # by the claim's bound on them (its winner budget)
                state._arena_prev = (prev, before, phase.claim_bound)
            for name, i in (("grown", 0), ("overflow", 1), ("needs_resort", 2)):
                state._defer_flag(name, out.flags, i)
            if out.flags.numel() > 4:
                state._defer_flag("tail_start", out.flags, 4)

    # -- generic passes (plastax_amd/generic.py) ---------------------------------
    def _generic_runner(self, which: str, g: Any) -> Any:
        from plastax_amd.generic import GenericPassRunner

        key = "_gen_" + which
        if getattr(self, key, None) is None:
            pp = self.plan.forward if which == "fwd" else self.plan.backward
            setattr(self, key, GenericPassRunner(pp.generic, self.static, g))
        return getattr(self, key)

    def _forward_generic(self, arena: Arena, units: dict, g: Any, stream: int) -> None:
        from plastax_amd import grow
        from plastax_amd.generic import finalize_lists

        run = self._generic_runner("fwd", g)
        k = grow.Kernels(arena.device, stream)
        fin = finalize_lists(arena, self.static)["fwd"]
        acc = run.new_acc(self.static.num_units, arena.device)
        for b in range(arena.num_buckets):
            rows = arena.fwd[b]
            run.fold(k, arena, b, units, acc, g, rows=rows.rows, nrows=rows.nrows, ptr=rows.ptr, entry_pos=None)
            if not arena.pipeline:
                run.apply(k, arena, units, acc, g, fin[b])
        if arena.pipeline:
            run.apply(k, arena, units, acc, g, fin[0])

    def _backward_generic(self, arena: Arena, units: dict, stream: int, g: Any) -> None:
        from plastax_amd import grow
        from plastax_amd.generic import finalize_lists

        run = self._generic_runner("bwd", g)
        k = grow.Kernels(arena.device, stream)
        fin = finalize_lists(arena, self.static)["bwd"]
        n = self.static.num_units
        acc = run.new_acc(n, arena.device)
        rows = torch.arange(n, dtype=torch.int32, device=arena.device)
        nb = arena.num_buckets
        churn = hasattr(arena, "lists")
        if arena.pipeline:
            if not churn:
                raise UnsupportedPolicyError("a generic backward on a PIPELINE net runs on the churn layout")
            lists = arena.lists[0]
            run.fold(k, arena, 0, units, acc, g, rows=rows, nrows=n, ptr=lists.ptr, entry_pos=lists.pos)
            run.apply(k, arena, units, acc, g, fin[0])
            return
        run.apply(k, arena, units, acc, g, fin[nb])
        for b in range(nb - 1, 0, -1):
            if churn:
                lists = arena.lists[b]
                run.fold(k, arena, b, units, acc, g, rows=rows, nrows=n, ptr=lists.ptr, entry_pos=lists.pos)
            else:  # the tiled layout: each source's out-edges in slot order from batch_sources
                from plastax_amd.batched import batch_sources

                bs = batch_sources(arena, b)
                run.fold(k, arena, b, units, acc, g, rows=bs.rows, nrows=bs.nrows, ptr=bs.ptr, entry_pos=bs.pos)
            run.apply(k, arena, units, acc, g, fin[b])

    # -- fused forward + prune (phases.py:1629-1848, :2322-2469) ---------------
    def _fusion_plan(self, g: Any) -> PruneFusionPlan:
        rec = self.prune_fusion
        if rec.plan is None:
            if self.plan.net.prune_conn is None:
                rec.plan = PruneFusionPlan(False, "no prune_conn")
            elif self.plan.forward.generic is not None:
                rec.plan = PruneFusionPlan(False, "the forward is a generic pass (no single-pass kernel)")
            elif rec.requested == "off":
                rec.plan = PruneFusionPlan(False, "fuse_prune='off'")
            else:
                rec.plan = plan_prune_fusion(self.plan.net, self.static, g, engine=rec.requested)
        return rec.plan

    def _fused_prune_progs(self, arena: Arena, units: dict, fin_common: dict, g: Any,
                           stream: int) -> list[torch.Tensor]:
        """The predicate's site program per bucket, in device memory, over
        the units the predicate sees (forwarded fields at their post-forward
        values); allocates the arena's sink column on first use."""
        from plastax_amd import grow

        if self._prune is None:
            self._prune = grow.PruneConnPhase(self.plan.net, self.static, g)
        if getattr(arena, "prune_sink", None) is None:
            arena.prune_sink = torch.zeros(arena.cols["dead"].numel(), dtype=torch.uint8, device=arena.device)
        pred_units = dict(units)
        names = self.prune_fusion.plan.forwarded
        if names:
            pred_units.update(self._forwarded(arena, units, fin_common, names, g, stream))
        self._pred_units = pred_units
        raws = []
        self._fused_handle = None
        for b in range(arena.num_buckets):
            base, cap = arena.bases[b], arena.caps[b]
            view = {name: col[base : base + cap] for name, col in arena.cols.items()}
            p = grow.fill_prog(self._prune.prog, pred_units, view, g, physical_ids=True)
            if b == 0 and FUSED_PREDICATE == "compiled":
                # (every bucket's program has the same code and field widths)
                self._fused_handle = grow.compiled_forward_prune_handle(self._prune.prog, p,
                                                                        self.plan.forward.monoid, arena.device)
            raws.append(bytes(memoryview(p).cast("B")))
        # One upload for every bucket's program, from pinned memory and
        # asynchronous on the step's stream (the programs hold this step's
        # globals, so they change every step; a synchronous copy would make
        # the host wait for the previous step's kernels).
        if not raws:
            return []
        size = -(-len(raws[0]) // 256) * 256
        host = torch.zeros(size * len(raws), dtype=torch.uint8, pin_memory=True)
        for b, raw in enumerate(raws):
            host[b * size : b * size + len(raw)] = torch.frombuffer(bytearray(raw), dtype=torch.uint8)
        dev_all = host.to(arena.device, non_blocking=True)  # (the current stream is the step's)
        return [dev_all[b * size : (b + 1) * size] for b in range(len(raws))]

    def _forwarded(self, arena: Arena, units: dict, fin_common: dict, names: tuple[str, ...], g: Any,
                   stream: int) -> dict[str, torch.Tensor]:
        """Post-forward values of the forwarded unit fields: the forward's
        apply from the identity accumulator on every unit the forward
        finalizes, the column's value elsewhere (phases.py:2367-2388)."""
        lib = _lib.load()
        fp = self.plan.forward
        n = self.static.num_units
        outs = {name: units[name].clone() for name in fp.program.out_fields if name is not None}
        prog = program_struct(fp.program, units, g, out_override=outs)
        if arena.pipeline:
            passes = [(torch.arange(n, dtype=torch.int32, device=arena.device), n, -1)]
        else:
            passes = [(arena.fwd[b].rows, arena.fwd[b].nrows, b + 1) for b in range(arena.num_buckets)]
        for rows, nrows, level in passes:
            if nrows == 0:
                continue
            parts = torch.arange(0, nrows + 256, 256, dtype=torch.int32, device=arena.device).clamp_(max=nrows)
            d = _lib.plx_partials_desc()
            d.nrows, d.monoid = nrows, fp.monoid
            d.nparts = -(-nrows // 256)
            d.part_rows = parts.data_ptr()
            d.row_unit = rows.data_ptr()
            d.fin.level, d.fin.is_input, d.fin.pruned = fin_common["level"], fin_common["is_input"], \
                fin_common["pruned"]
            d.fin.fin_level, d.fin.skip_inputs = level, 1
            d.apply = prog
            _lib.check(lib.plx_backward_partials(d, stream), "plx_backward_partials")
        return {name: outs[name] for name in names}

    def _xla_prune(self, arena: Arena, g: Any, stream: int) -> None:
        """The "xla" engine: the predicate pass at the forward's slot, into
        the sink (two reads of the edge columns, one phase)."""
        from plastax_amd import grow

        k = grow.Kernels(arena.device, stream)
        arena.prune_sink.zero_()
        n_units = self.static.num_units
        for b in range(arena.num_buckets):
            base, cap = arena.bases[b], arena.caps[b]
            if cap == 0:
                continue
            view = {name: col[base : base + cap] for name, col in arena.cols.items()}
            k.site_eval(self._prune.prog, self._pred_units, g, n=cap, kind=5, num_units=n_units, conns=view,
                        or_into=arena.prune_sink[base : base + cap], site_ids=arena.slot[base : base + cap],
                        ids_logical=arena.uperm32, ids_physical=arena.uinv32)

    def _merge_prune(self, arena: Arena, stream: int) -> None:
        """Commit the fused forward's tombstones (phases.py:2447-2469)."""
        lib = _lib.load()
        sink, dead = arena.prune_sink, arena.cols["dead"]
        for b in range(arena.num_buckets):
            base, cap = arena.bases[b], arena.caps[b]
            if cap == 0:
                continue
            stamp, value = arena.stamp_target(b)
            _lib.check(lib.plx_merge_kills(cap, sink[base:].data_ptr(), dead[base:].data_ptr(),
                                           None if stamp is None else stamp.data_ptr(), float(value), stream),
                       "plx_merge_kills")

    # -- phases -----------------------------------------------------------------
    @staticmethod
    def _shadow(units: dict[str, torch.Tensor], out_fields: list[str | None]) -> dict[str, torch.Tensor]:
        """PIPELINE applies write every unit at once against the pre-phase
        columns (sweep.py:205-228): write into copies, swapped in after."""
        return {f: units[f].clone() for f in out_fields if f is not None}

    @staticmethod
    def _unshadow(units: dict[str, torch.Tensor], swaps: dict[str, torch.Tensor]) -> None:
        for name, buf in swaps.items():
            units[name] = buf

    def _loss(self, plan: Plan, units: dict, inputs: StepInputs, consts: dict,
              loss: torch.Tensor, stream: int, g: Any) -> None:
        lib = _lib.load()
        dev = loss.device
        n_out = len(self.static.output_ids)
        if inputs.targets is None:
            raise ValueError("step: this net has a loss, so StepInputs.targets is required")
        t = torch.as_tensor(inputs.targets, dtype=torch.float32, device=dev).reshape(-1).contiguous()
        if t.numel() != n_out:
            raise ValueError(f"step: expected {n_out} targets, got {t.numel()}")
        lp = plan.loss
        seed = units[lp.seed_field]
        if lp.kind == "softmax":
            _lib.check(
                lib.plx_loss_softmax_ce(
                    n_out,
                    consts["output_ids"].data_ptr(),
                    units[ACTIVATION.name].data_ptr(),
                    t.data_ptr(),
                    seed.data_ptr(),
                    loss.data_ptr(),
                    stream,
                ),
                "plx_loss_softmax_ce",
            )
            return
        scratch = torch.empty(n_out // 256 + 2, dtype=torch.float32, device=dev)
        prog = program_struct(lp.program, units, g, unit_map=consts["unit_map"])
        _lib.check(
            lib.plx_loss_elementwise(
                n_out,
                consts["output_ids"].data_ptr(),
                t.data_ptr(),
                prog,
                seed.data_ptr(),
                scratch.data_ptr(),
                loss.data_ptr(),
                stream,
            ),
            "plx_loss_elementwise",
        )

    def _tiles(self, plan: Plan, arena: Arena, units: dict, consts: dict, b: int,
               fold: bool, update: bool, stream: int) -> None:
        lib = _lib.load()
        bt = arena.bwd[b]
        if arena.lives[b] == 0:
            return  # no edge was live when the arena was laid out: nothing to fold or update
        d = _lib.plx_tile_desc()
        d.base = bt.base
        d.end = bt.end
        d.tile_size = arena.tile
        d.ntiles = bt.ntiles
        d.nsuper = bt.nsuper
        d.tile_pos = bt.tile_pos.data_ptr()
        d.super_tile = bt.super_tile.data_ptr()
        d.fold = int(fold)
        d.update = int(update)
        d.src = arena.cols["from_id"].data_ptr()
        d.dst = arena.cols["to_id"].data_ptr()
        d.dead = arena.cols["dead"].data_ptr()
        d.weight = arena.cols["weight"].data_ptr()
        if fold:
            bp = plan.backward
            d.monoid = bp.monoid
            d.nhot = bt.nhot
            d.hot_base = bt.hot_base
            d.tile_info = bt.tile_info.data_ptr()
            d.grp_off = bt.grp_off.data_ptr()
            d.grp = bt.grp.data_ptr()
            if arena.dst8[b] is not None:
                d.dst8 = arena.dst8[b].data_ptr()
                d.blk_dst0 = arena.blk_dst0[b].data_ptr()
            d.sorted_rank = bt.sorted_rank.data_ptr()
            d.hot_sb = bt.hot_sb.data_ptr()
            d.cold_partial = bt.cold_partial.data_ptr()
            d.g = bp.gathered(units, ACTIVATION.name).data_ptr()
            d.map = bp.map_struct()
        if update:
            up = plan.update
            d.rule = up.rule_code
            d.tbl_base, d.tbl_len = arena.src_table(b)
            for k, name in enumerate(up.state_columns()):
                setattr(d, f"s{k}", arena.cols[name].data_ptr())
            d.gfield = units[up.grad_field.name].data_ptr()
            d.act = units[ACTIVATION.name].data_ptr()
            if "pow_table" in consts:
                d.pow_table = consts["pow_table"].data_ptr()
                d.pow_table_len = consts["pow_table"].numel() // 2
            for k, v in enumerate(up.params()):
                d.p[k] = float(v)
        self._edge_state(d, arena, b, update)
        kind = "backward_update" if fold and update else ("backward" if fold else "update_conn")
        self._launch(kind, lib.plx_backward_tiles, d, stream)
        if update:
            self._advance_t(arena, b)

    def _partials(self, plan: Plan, bt: Any, acc: Any, prog: Any, fin_common: dict,
                  fin_level: int, skip_inputs: int, stream: int) -> None:
        lib = _lib.load()
        d = _lib.plx_partials_desc()
        d.nrows = bt.nrows
        d.monoid = plan.backward.monoid
        d.nsuper = bt.nsuper
        d.nhot = bt.nhot
        d.nparts = bt.nparts
        d.part_rows = bt.part_rows.data_ptr() if bt.part_rows is not None else None
        d.part_info = bt.part_info.data_ptr() if bt.part_info is not None and bt.row_hot is not None else None
        d.row_unit = bt.rows.data_ptr()
        if bt.row_hot is not None:
            d.row_hot = bt.row_hot.data_ptr()
            d.row_cold = bt.row_cold.data_ptr()
            d.hot_sb = bt.hot_sb.data_ptr()
            d.cold_partial = bt.cold_partial.data_ptr()
            d.cold_sb = bt.cold_sb.data_ptr()
            d.cold_idx = bt.cold_idx.data_ptr()
        d.acc = acc.data_ptr() if acc is not None else None
        d.fin.level = fin_common["level"]
        d.fin.is_input = fin_common["is_input"]
        d.fin.pruned = fin_common["pruned"]
        d.fin.fin_level = fin_level
        d.fin.skip_inputs = skip_inputs
        d.apply = prog
        self._launch("backward_finalize", lib.plx_backward_partials, d, stream)

    def _backward_lists(self, plan: Plan, arena: Any, units: dict, fin_common: dict, stream: int,
                        g: Any) -> None:
        """The churn layout's backward: per bucket, every unit a row folding
        its live out-edges in slot order (sweep.py:343-449)."""
        lib = _lib.load()
        bp = plan.backward
        dev = arena.device
        n = self.static.num_units
        nb = arena.num_buckets
        swaps = self._shadow(units, bp.program.out_fields) if arena.pipeline else {}
        acc = torch.empty(n, dtype=torch.float32, device=dev)
        _lib.call("plx_fill_f32", n, bp.identity, acc.data_ptr(), stream)
        prog = program_struct(bp.program, units, g, out_override=swaps)
        rows = arena.fwd[0].rows

        def run(lists: Any, level: int, skip_inputs: int) -> None:
            d = _lib.plx_bwd_batch_desc()
            d.nrows = n
            d.monoid = bp.monoid
            d.batch = 1
            d.row_unit = rows.data_ptr()
            if lists is None:
                zeros = torch.zeros(n + 1, dtype=torch.int32, device=dev)
                d.row_ptr = zeros.data_ptr()
                d.dst = zeros.data_ptr()
                d.weight = acc.data_ptr()
                d.live = None
            else:
                # Only what the pass reads: the weights unless the map holds
                # them constant, liveness while tombstones sit in the lists.
                need_w = bp.w_const is None
                need_live = arena.dead_in_rows
                if need_w or need_live:
                    _lib.check(lib.plx_gather_edges(
                        lists.pos.numel(), lists.pos.data_ptr(), arena.cols["weight"].data_ptr(),
                        arena.cols["dead"].data_ptr(), lists.weight.data_ptr() if need_w else None,
                        lists.live.data_ptr() if need_live else None, stream), "plx_gather_edges")
                d.row_ptr = lists.ptr.data_ptr()
                d.dst = lists.dst.data_ptr()
                d.weight = lists.weight.data_ptr()
                d.live = lists.live.data_ptr() if need_live else None
            d.g = bp.gathered(units, ACTIVATION.name).data_ptr()
            d.map = bp.map_struct()
            d.acc = acc.data_ptr()
            d.fin.level = fin_common["level"]
            d.fin.is_input = fin_common["is_input"]
            d.fin.pruned = fin_common["pruned"]
            d.fin.fin_level = level
            d.fin.skip_inputs = skip_inputs
            d.apply = prog
            self._launch("backward", lib.plx_backward_lists, d, stream)

        if arena.pipeline:
            run(arena.lists[0], -1, 0)
        else:
            run(None, nb, 1)
            for b in range(nb - 1, 0, -1):
                run(arena.lists[b], b, 1)
        self._unshadow(units, swaps)

    def _backward_update(self, plan: Plan, arena: Arena, units: dict, consts: dict,
                         fin_common: dict, stream: int, g: Any) -> None:
        bp, up = plan.backward, plan.update
        nb = arena.num_buckets
        # (a generic backward is its own pass on either layout; the update
        # then runs bucket by bucket on its own)
        if getattr(arena, "churn", False) or (bp is not None and bp.generic is not None):
            if bp is not None and bp.generic is not None:
                self._backward_generic(arena, units, stream, g)
            elif bp is not None:
                self._backward_lists(plan, arena, units, fin_common, stream, g)
            if plan.update_unit:
                self._run_update_unit(arena, units, stream, g)
            if up is not None:
                for b in range(nb):
                    self._update_only(plan, arena, units, consts, b, stream)
            if plan.update_generic:
                self._run_update_generic(arena, units, stream, g)
            return
        if bp is not None:
            dev = arena.device
            n_units = self.static.num_units
            swaps = self._shadow(units, bp.program.out_fields) if arena.pipeline else {}
            acc = None
            if arena.bwd_carry:
                acc = torch.empty(n_units, dtype=torch.float32, device=dev)
                _lib.call("plx_fill_f32", n_units, bp.identity, acc.data_ptr(), stream)
            prog = program_struct(bp.program, units, g, out_override=swaps)
            if arena.pipeline:
                # One sweep reading the pre-phase grads; every unit, inputs
                # included, is applied (sweep.py:442-447). The update then
                # reads the new grads, so it is its own pass.
                self._tiles(plan, arena, units, consts, 0, True, False, stream)
                self._partials(plan, arena.bwd[0], acc, prog, fin_common, -1, 0, stream)
            else:
                # update_unit runs between the backward and update_conn
                # (phases.py:87-182), so with one the passes are not fused.
                fused = up is not None and not plan.update_unit
                self._partials(plan, arena.top, acc, prog, fin_common, nb, 1, stream)
                for b in range(nb - 1, 0, -1):
                    self._tiles(plan, arena, units, consts, b, True, fused, stream)
                    self._partials(plan, arena.bwd[b], acc, prog, fin_common, b, 1, stream)
            self._unshadow(units, swaps)
        if plan.update_unit:
            self._run_update_unit(arena, units, stream, g)
        if up is not None:
            if bp is None or arena.pipeline or plan.update_unit:
                todo = range(nb)
            else:
                todo = range(1)  # bucket 0 is never reduced, only updated
            for b in todo:
                self._update_only(plan, arena, units, consts, b, stream)
        if plan.update_generic:
            self._run_update_generic(arena, units, stream, g)

    def _run_update_generic(self, arena: Arena, units: dict, stream: int, g: Any) -> None:
        """A user UpdateConn (phases.py:1196-1242): incoming over every bucket,
        then outgoing, as edge programs on the physical arena."""
        from plastax_amd import grow

        if self._update_generic is None:
            self._update_generic = grow.ConnUpdatePhase(self.plan.net, self.static, g)
        self._update_generic.run_physical(grow.Kernels(arena.device, stream), arena, units, g)

    def _run_update_unit(self, arena: Arena, units: dict, stream: int, g: Any) -> None:
        """update_unit (phases.py:1148-1193) on the step's unit columns, in the
        arena's unit order (the program sees the caller's ids)."""
        from plastax_amd import grow, units as unit_phases

        if self._update_unit is None:
            self._update_unit = unit_phases.UpdateUnitPhase(self.plan.net, self.static, g)
        k = grow.Kernels(arena.device, stream)
        self._update_unit.run(k, units, g, site_ids=arena.uperm32, ids_physical=arena.uinv32)

    def _update_only(self, plan: Plan, arena: Arena, units: dict, consts: dict, b: int,
                     stream: int) -> None:
        """A bucket the walk never reduces: the update rule alone, one 16-byte
        quad of positions per lane (phases.py:1196-1242)."""
        lib = _lib.load()
        up = plan.update
        base, end = arena.bases[b], arena.ends[b]
        d = _lib.plx_update_desc()
        d.n = end - base
        d.rule = up.rule_code
        d.tbl_base, d.tbl_len = arena.src_table(b)

        def col(name: str) -> int:
            t = arena.cols[name]
            return t.data_ptr() + base * t.element_size()

        d.src = col("from_id")
        d.dst = col("to_id")
        d.dead = col("dead")
        d.weight = col("weight")
        for k, name in enumerate(up.state_columns()):
            setattr(d, f"s{k}", col(name))
        d.gfield = units[up.grad_field.name].data_ptr()
        d.act = units[ACTIVATION.name].data_ptr()
        if "pow_table" in consts:
            d.pow_table = consts["pow_table"].data_ptr()
            d.pow_table_len = consts["pow_table"].numel() // 2
        for k, v in enumerate(up.params()):
            d.p[k] = float(v)
        if arena.dst8[b] is not None:
            d.dst8 = arena.dst8[b].data_ptr()
            d.blk_dst0 = arena.blk_dst0[b].data_ptr()
        self._edge_state(d, arena, b, True)
        # positions of this descriptor start at the bucket base
        d.live_end -= base
        d.dead = col("dead") if arena.dead_in_rows else None
        self._launch("update_conn", lib.plx_update_conn, d, stream)
        self._advance_t(arena, b)
