"""The batched step: ``make_step(net, static, batch_size=B)``.

Mirrors src/plastax/step.py:359-468 and phases.py:217-532. Forward, loss and
backward run once per sample against the shared connections; the connection
update is one optimizer step on the batch-mean gradient (the optim bundles'
exact ``per_sample`` / ``incoming_batched`` pair, phases.py:434-483); the
per-sample unit columns are reduced by the network's ``batch_reduction``
(phases.py:298-332); the structural phases then run once on the reduced
state, and ``StepResult.loss`` is the batch mean.

Device layout: during the step every unit column a per-sample phase reads or
writes is a ``[num_units, B]`` tensor (sample b of unit u at ``u * B + b``),
in the arena's physical unit order. A forward row (destination) or a backward
row (source) is one workgroup whose lanes are the samples: the gathered unit
row is one coalesced B-wide read and the edge columns are uniform across the
workgroup. Summation orders, per sample:

- forward: a destination's live in-edges in slot order (the streaming
  step's, so a batch of one equals the streaming forward bit for bit);
- backward: a source's live out-edges in logical slot order, from the
  identity (the reference's per-sample scatter order);
- update: ``stat_0 + stat_1 + ... + stat_{B-1}`` then ``/ B``
  (phases.py:462-471);
- MEAN / SUM reductions: samples in order from sample 0; the loss mean
  ``(0 + l_0 + ... ) / B``.
"""

from __future__ import annotations

import ctypes
from typing import Any

import numpy as np
import torch

from plastax_amd import _layout, _lib
from plastax_amd._expr import UnsupportedPolicyError
from plastax_amd._layout import Arena
from plastax_amd._plan import Plan, program_struct
from plastax_amd._types import ACTIVATION
from plastax_amd.state import NetworkState, NetworkStatic
from plastax_amd.step import StepFn, StepInputs, StepResult, _stream
from plastax_amd.traits import Reduction, batch_written_reduction

_REDUCE = {Reduction.MEAN: 0, Reduction.SUM: 1, Reduction.FIRST: 2}


class BatchSources:
    """Per bucket, its backward rows (sources) and their out-edge lists in
    logical slot order: list entry j (``ptr[r] <= j < ptr[r+1]``) is physical
    position ``pos[j]``, whose TO_ID ``dst[j]`` is fixed with the layout; the
    step gathers the entries' weights and liveness into ``weight`` / ``live``
    (one wide gather), so the backward reads every list sequentially."""

    def __init__(self, nrows: int, rows: torch.Tensor, ptr: torch.Tensor, pos: torch.Tensor,
                 dst: torch.Tensor) -> None:
        self.nrows = nrows
        self.rows = rows
        self.ptr = ptr
        self.pos = pos
        self.dst = dst
        n = int(pos.numel())
        self.weight = torch.empty(n, dtype=torch.float32, device=pos.device)
        self.live = torch.empty(n, dtype=torch.uint8, device=pos.device)


def batch_sources(arena: Arena, b: int) -> BatchSources:
    """Bucket b's backward rows: every unit of level b and every live source
    of the bucket, ascending; each row's live positions sorted by logical slot
    (built on the device, cached on the arena, whose structure it follows)."""
    from plastax_amd._batch_dev import batch_sources_dev

    cache = arena.__dict__.setdefault("_batch_sources", {})
    if b not in cache:
        cache[b] = batch_sources_dev(arena, b)
    return cache[b]


def batch_sources_host(arena: Arena, b: int) -> BatchSources:
    """batch_sources built on the host with numpy (the restatement the
    device build is tested against)."""
    base, live = arena.bases[b], arena.lives[b]
    src = arena.cols["from_id"][base : base + live].cpu().numpy().astype(np.int64)
    dst_all = arena.cols["to_id"][base : base + live].cpu().numpy().astype(np.int64)
    slot = arena.slot[base : base + live].cpu().numpy().astype(np.int64)
    if b + 1 < arena.lvl_start.size:
        level_units = np.arange(int(arena.lvl_start[b]), int(arena.lvl_start[b + 1]), dtype=np.int64)
    else:
        level_units = np.zeros(0, dtype=np.int64)  # no unit has this level
    rows = np.union1d(level_units, np.unique(src))
    order = np.lexsort((slot, src))
    pos = (order + base).astype(np.int64)
    ptr = np.searchsorted(src[order], rows, side="left")
    ptr = np.concatenate([ptr, [live]]).astype(np.int64)
    dev = arena.device
    out = BatchSources(
        int(rows.size),
        torch.from_numpy(rows.astype(np.int32)).to(dev),
        torch.from_numpy(ptr.astype(np.int32)).to(dev),
        torch.from_numpy(np.concatenate([pos, [base]]).astype(np.int32)).to(dev),
        torch.from_numpy(np.concatenate([dst_all[order], [0]]).astype(np.int32)).to(dev),
    )
    return out


def written_columns(plan: Plan, static: NetworkStatic, update_unit: list[str] = (),
                    forward_generic: list[str] = (), backward_generic: list[str] = ()) -> dict[str, str]:
    """The unit columns a batched step's per-sample phases write, each with
    the first phase writing it (phases.py:334-387); ``update_unit`` names the
    columns the traced update_unit writes, ``forward_generic`` /
    ``backward_generic`` those a generic pass's apply writes."""
    written = {ACTIVATION.name: "the input scatter"}
    for name in list(plan.forward.program.out_fields) + list(forward_generic):
        if name is not None:
            written.setdefault(name, "forward_pass")
    if plan.loss is not None:
        written.setdefault(plan.loss.seed_field, "loss")
    if plan.backward is not None:
        for name in list(plan.backward.program.out_fields) + list(backward_generic):
            if name is not None:
                written.setdefault(name, "backward_pass")
    for name in update_unit:
        written.setdefault(name, "update_unit")
    return written


class BatchedStepFn(StepFn):
    """The callable ``make_step(..., batch_size=B)`` returns."""

    def __init__(self, plan: Plan, static: NetworkStatic, batch_size: int) -> None:
        super().__init__(plan, static)
        self.batch = int(batch_size)
        self.arena_mode = "tiled"  # the batched kernels read the tiled layout's forward rows

    def churn(self) -> bool:
        return False  # a generic backward reads batch_sources' lists, which the tiled layout has

    def _generic_runners(self, g: Any) -> list[Any]:
        """The traced generic passes (forward, backward), None where the pass
        has the product form (traced on the first call, against ``g``)."""
        out = []
        for which, pp in (("fwd", self.plan.forward), ("bwd", self.plan.backward)):
            out.append(self._generic_runner(which, g) if pp is not None and pp.generic else None)
        return out

    def _check_policy(self, g: Any) -> dict[str, Reduction]:
        """Every column a per-sample phase writes has a MEAN / SUM / FIRST
        reduction (step.py:429-441); returns them."""
        net = self.plan.net
        policy = net.batch_reduction
        specs = {s.name: s for s in self.static.unit_fields}
        out = {}
        uu = self._update_unit.names if self._update_unit is not None else []
        gf, gb = self._generic_runners(g)
        gen = [list(r.names) if r is not None else [] for r in (gf, gb)]
        for name, where in written_columns(self.plan, self.static, uu, *gen).items():
            try:
                out[name] = batch_written_reduction(policy, specs[name], where=where)
            except ValueError as err:
                raise ValueError(f"{net.__name__}.{err}") from None
        return out

    def _batched_columns(self, units: dict[str, torch.Tensor], g: Any) -> dict[str, torch.Tensor]:
        """[num_units, B] copies of every column a per-sample phase reads or
        writes (each sample starts from the shared state: step.py:421-424)."""
        plan = self.plan
        names = {ACTIVATION.name} | ({plan.forward.field} - {None})
        progs = [plan.forward.program]
        if plan.loss is not None:
            names.add(plan.loss.seed_field)
            if plan.loss.program is not None:
                progs.append(plan.loss.program)
        if plan.backward is not None:
            if plan.backward.field is not None:
                names.add(plan.backward.field)
            progs.append(plan.backward.program)
        if plan.update is not None:
            names.add(plan.update.grad_field.name)
        if self._update_unit is not None:
            names.update(self._update_unit.prog.unit_fields)
            names.update(self._update_unit.names)
        if self._update_generic is not None:
            for prog, _ in self._update_generic.passes:
                names.update(prog.unit_fields)
        for run in self._generic_runners(g):
            if run is not None:
                names.update(run.map_prog.unit_fields)
                names.update(n for n in run.apply_prog.unit_fields if n not in run.acc_names)
                names.update(run.names)
        names.discard("pruned")
        for p in progs:
            names.update(n for n in p.fields)
            names.update(n for n in p.out_fields if n is not None)
        B = self.batch
        return {n: units[n].unsqueeze(1).expand(-1, B).contiguous() for n in sorted(names)}

    def __call__(self, state: NetworkState, inputs: StepInputs) -> StepResult:
        from plastax_amd import grow
        from plastax_amd.generic import finalize_lists

        plan = self.plan
        B = self.batch
        dev = state.device
        if dev.type != "cuda":
            raise RuntimeError("the plastax_amd step runs on a GPU; the state lives on the CPU")
        n_in, n_out = len(self.static.input_ids), len(self.static.output_ids)
        x = torch.as_tensor(inputs.inputs, dtype=torch.float32, device=dev)
        if tuple(x.shape) != (B, n_in):
            raise ValueError(f"batched step: inputs must be {(B, n_in)}, got {tuple(x.shape)}")
        t = None
        if inputs.targets is not None:
            t = torch.as_tensor(inputs.targets, dtype=torch.float32, device=dev)
            if tuple(t.shape) != (B, n_out):
                raise ValueError(f"batched step: targets must be {(B, n_out)}, got {tuple(t.shape)}")
            t = t.contiguous()
        if plan.update_unit and self._update_unit is None:
            from plastax_amd import units as unit_phases

            self._update_unit = unit_phases.UpdateUnitPhase(plan.net, self.static, state.globals_)
        if plan.update_generic and self._update_generic is None:
            from plastax_amd import grow

            self._update_generic = grow.ConnUpdatePhase(plan.net, self.static, state.globals_)
        reductions = self._check_policy(state.globals_)
        lib = _lib.load()
        state = state._donate()
        arena = self.arena(state)
        consts = self._consts(dev, arena)
        stream = _stream(dev)
        units = state._physical_units(arena)
        n_units = self.static.num_units
        g = state.globals_
        ub = self._batched_columns(units, g)
        if n_in:
            ub[ACTIVATION.name][consts["input_ids"].long()] = x.t()
        fin = dict(
            level=units["level"].data_ptr(),
            is_input=consts["is_input"].data_ptr(),
            pruned=units["pruned"].data_ptr() if "pruned" in units else None,
        )

        gf, gb = self._generic_runners(g)
        if (gf is not None or gb is not None) and arena.pipeline:
            raise UnsupportedPolicyError("a batched step runs generic passes on level-synchronous nets only")
        pruned = units.get("pruned")

        # Forward, per sample (phases.py:942-1015; step.py:443-447).
        fp = plan.forward
        acc = None
        if gf is not None:
            gf.check_columns(ub, B)
            k = grow.Kernels(dev, stream)
            fin_lists = finalize_lists(arena, self.static)["fwd"]
            gacc = gf.new_acc(n_units, dev, B)
            for b in range(arena.num_buckets):
                rows = arena.fwd[b]
                gf.fold(k, arena, b, ub, gacc, g, rows=rows.rows, nrows=rows.nrows, ptr=rows.ptr, entry_pos=None,
                        batch=B)
                gf.apply(k, arena, ub, gacc, g, fin_lists[b], batch=B, pruned=pruned)
        elif arena.fwd_carry:
            acc = torch.full((n_units, B), fp.identity, dtype=torch.float32, device=dev)
        prog = program_struct(fp.program, ub, g)
        for b in range(arena.num_buckets if gf is None else 0):
            rows = arena.fwd[b]
            d = _lib.plx_forward_desc()
            d.nrows = rows.nrows
            d.monoid = fp.monoid
            d.row_unit = rows.rows.data_ptr()
            d.row_ptr = rows.ptr.data_ptr()
            d.src = arena.cols["from_id"].data_ptr()
            d.weight = arena.cols["weight"].data_ptr()
            d.dead = arena.cols["dead"].data_ptr() if arena.dead_in_rows else None
            d.x = fp.gathered(ub, ACTIVATION.name).data_ptr()
            d.map = fp.map_struct()
            d.acc = acc.data_ptr() if acc is not None else None
            d.fin.level, d.fin.is_input, d.fin.pruned = fin["level"], fin["is_input"], fin["pruned"]
            d.fin.fin_level = b + 1
            d.fin.skip_inputs = 1
            d.apply = prog
            self._launch("forward", lib.plx_forward_batch, d, B, stream)

        # Loss, per sample, then the batch mean (step.py:448-451, :466).
        loss = torch.zeros((), dtype=torch.float32, device=dev)
        if plan.loss is not None:
            if t is None:
                raise ValueError("step: this net has a loss, so StepInputs.targets is required")
            losses = torch.empty(B, dtype=torch.float32, device=dev)
            lp = plan.loss
            ids = consts["output_ids"].data_ptr()
            if lp.kind == "softmax":
                _lib.check(
                    lib.plx_loss_softmax_ce_batch(n_out, ids, ub[ACTIVATION.name].data_ptr(), t.data_ptr(),
                                                  ub[lp.seed_field].data_ptr(), losses.data_ptr(), B, stream),
                    "plx_loss_softmax_ce_batch",
                )
            else:
                parts = torch.empty(B * (n_out // 256 + 1) + 1, dtype=torch.float32, device=dev)
                lprog = program_struct(lp.program, ub, g, batch=B, unit_map=consts["unit_map"])
                _lib.check(
                    lib.plx_loss_elementwise_batch(n_out, ids, t.data_ptr(), lprog, ub[lp.seed_field].data_ptr(),
                                                   parts.data_ptr(), losses.data_ptr(), B, stream),
                    "plx_loss_elementwise_batch",
                )
            _lib.check(lib.plx_batch_mean(B, losses.data_ptr(), loss.data_ptr(), stream), "plx_batch_mean")

        # Backward, per sample (phases.py:1049-1104): the deepest level from
        # the identity, then buckets L-1 .. 1 in the reference's slot order.
        bp = plan.backward
        if gb is not None:
            gb.check_columns(ub, B)
            k = grow.Kernels(dev, stream)
            fin_lists = finalize_lists(arena, self.static)["bwd"]
            gacc = gb.new_acc(n_units, dev, B)
            nb = arena.num_buckets
            gb.apply(k, arena, ub, gacc, g, fin_lists[nb], batch=B, pruned=pruned)
            for b in range(nb - 1, 0, -1):
                lists = batch_sources(arena, b)
                gb.fold(k, arena, b, ub, gacc, g, rows=lists.rows, nrows=lists.nrows, ptr=lists.ptr,
                        entry_pos=lists.pos, batch=B)
                gb.apply(k, arena, ub, gacc, g, fin_lists[b], batch=B, pruned=pruned)
        elif bp is not None:
            bacc = None
            if arena.bwd_carry:
                bacc = torch.full((n_units, B), bp.identity, dtype=torch.float32, device=dev)
            bprog = program_struct(bp.program, ub, g)
            empty = torch.zeros(1, dtype=torch.int32, device=dev)

            def run(rows: torch.Tensor, nrows: int, ptr: torch.Tensor, lists: Any, level: int) -> None:
                d = _lib.plx_bwd_batch_desc()
                d.nrows = nrows
                d.monoid = bp.monoid
                d.batch = B
                d.row_unit = rows.data_ptr()
                d.row_ptr = ptr.data_ptr()
                d.dst = lists.dst.data_ptr()
                d.weight = lists.weight.data_ptr()
                d.live = lists.live.data_ptr()
                d.g = bp.gathered(ub, ACTIVATION.name).data_ptr()
                d.map = bp.map_struct()
                d.acc = bacc.data_ptr() if bacc is not None else None
                d.fin.level, d.fin.is_input, d.fin.pruned = fin["level"], fin["is_input"], fin["pruned"]
                d.fin.fin_level = level
                d.fin.skip_inputs = 1
                d.apply = bprog
                self._launch("backward", lib.plx_backward_batch, d, stream)

            nb = arena.num_buckets
            top = arena.top
            if top.nrows:
                zeros = torch.zeros(top.nrows + 1, dtype=torch.int32, device=dev)
                none = BatchSources(0, empty, empty, empty, empty)
                run(top.rows, top.nrows, zeros, none, nb)
            for b in range(nb - 1, 0, -1):
                lists = batch_sources(arena, b)
                # This step's (pre-update) weights and tombstones, in slot order.
                _lib.check(
                    lib.plx_gather_edges(lists.pos.numel(), lists.pos.data_ptr(), arena.cols["weight"].data_ptr(),
                                         arena.cols["dead"].data_ptr(), lists.weight.data_ptr(),
                                         lists.live.data_ptr(), stream),
                    "plx_gather_edges",
                )
                run(lists.rows, lists.nrows, lists.ptr, lists, b)

        # update_unit, per sample (step.py:435-436), on the live units.
        if plan.update_unit:
            skip = None
            if "pruned" in units:
                skip = units["pruned"].unsqueeze(1).expand(-1, B).contiguous()
            self._update_unit.run(grow.Kernels(dev, stream), ub, g, site_ids=arena.uperm32,
                                  ids_physical=arena.uinv32, batch=B, skip=skip)

        # The connection update on the batch-mean gradient (phases.py:434-483).
        up = plan.update
        if up is not None:
            for b in range(arena.num_buckets):
                self._update_batch(plan, arena, ub, consts, b, stream)
            state._mark_ahead()
        if plan.update_generic:
            self._mean_of_writes(arena, ub, g, stream)
            state._mark_ahead()

        # reduce_batch_units (phases.py:298-332): the written columns only.
        for name, red in reductions.items():
            col = units[name]
            kind = 0 if col.dtype == torch.float32 else (1 if col.dtype == torch.int32 else 2)
            _lib.check(
                lib.plx_reduce_batch(n_units, B, _REDUCE[red], kind, ub[name].data_ptr(), col.data_ptr(), stream),
                "plx_reduce_batch",
            )

        # Once per batch: structural phases and reset_global (step.py:455-459).
        if plan.prune_unit or plan.prune_conn or plan.add_unit or plan.add_conn is not None:
            self._structural(state, arena, units, stream, g)
        if plan.reset_global:
            state.globals_ = plan.net.reset_global.reset(state.globals_)
        state.step = state.step + 1
        return StepResult(state=state, overflow=state._flag_reader("overflow"), loss=loss, growth_remainder=None)

    def _mean_of_writes(self, arena: Arena, ub: dict, g: Any, stream: int) -> None:
        """A user UpdateConn under a batched step (phases.py:484-533): each
        sample's incoming then outgoing pass against the unchanged
        connections; every float32 column's per-sample changes are summed in
        sample order and old + total / B is kept, a non-float column takes
        sample 0's write. A float column neither pass writes has the change
        old - old for every sample (+0, or NaN where old is not finite), so
        its total is the first one and one APPLY gives the result."""
        from plastax_amd import grow

        lib = _lib.load()
        B = self.batch
        k = grow.Kernels(arena.device, stream)
        passes = self._update_generic.passes
        written = sorted({n for _, names in passes for n in names})
        n_units = int(next(iter(ub.values())).shape[0])
        for b in range(arena.num_buckets):
            base, cap, live = arena.bases[b], arena.caps[b], arena.lives[b]
            if cap == 0:
                continue
            old = {name: col[base : base + cap] for name, col in arena.cols.items()}
            floats = [n for n, c in old.items() if c.dtype == torch.float32]
            total = {n: torch.empty_like(old[n]) for n in floats}
            first = {}
            for s in range(B):
                work = {n: old[n].clone() for n in written}
                view = {n: work.get(n, old[n]) for n in old}
                for prog, names in passes:
                    if names and live:
                        k.site_eval(prog, ub, g, n=live, kind=grow._lib_sites("EDGE"), num_units=n_units,
                                    conns={n: c[:live] for n, c in view.items()},
                                    outs=[view[n][:live] for n in names],
                                    from_id=view["from_id"][:live], to_id=view["to_id"][:live],
                                    site_ids=arena.slot[base : base + live], ids_logical=arena.uperm32,
                                    ids_physical=arena.uinv32, batch=B, sample=s)
                for n in floats:
                    if n not in written and s > 0:
                        continue
                    mode = _lib.PLX_MOW_FIRST if s == 0 else _lib.PLX_MOW_ADD
                    _lib.check(lib.plx_mean_of_writes(cap, mode, B, old[n].data_ptr(), view[n].data_ptr(),
                                                      total[n].data_ptr(), stream), "plx_mean_of_writes")
                if s == 0:
                    first = {n: work[n] for n in written if old[n].dtype != torch.float32}
            for n in floats:
                _lib.check(lib.plx_mean_of_writes(cap, _lib.PLX_MOW_APPLY, B, old[n].data_ptr(), None,
                                                  total[n].data_ptr(), stream), "plx_mean_of_writes")
            for n, w in first.items():
                old[n].copy_(w)

    def _update_tiles(self, arena: Arena, b: int) -> tuple[Any, tuple]:
        """Bucket b's batched-update tiles (built once per arena): the edges
        grouped by 64 destination x 64 source units, so a workgroup stages
        their unit rows in LDS."""
        cache = arena.__dict__.setdefault("_batch_tiles", {})
        if not cache:
            rows, edges = ctypes.c_int32(), ctypes.c_int32()
            _lib.check(_lib.load().plx_batch_tile_limits(ctypes.byref(rows), ctypes.byref(edges)),
                       "plx_batch_tile_limits")
            if (rows.value, edges.value) != (_layout.BATCH_TILE_UNITS, _layout.BATCH_TILE_EDGES):
                raise RuntimeError(
                    f"the library's batched-update tiles are {rows.value} units / {edges.value} edges, "
                    f"the layout builds {_layout.BATCH_TILE_UNITS} / {_layout.BATCH_TILE_EDGES}: rebuild it")
        if b not in cache:
            from plastax_amd._batch_dev import batch_tiles_dev

            cache[b] = batch_tiles_dev(arena, b)
        c = cache[b]
        t = _lib.plx_batch_tiles()
        t.ntiles = int(c["tile_off"].numel()) - 1
        t.num_units = self.static.num_units
        t.tile_off = c["tile_off"].data_ptr()
        t.tile_base = c["tile_base"].data_ptr()
        t.pos = c["pos"].data_ptr()
        t.loc = c["loc"].data_ptr()
        return t, (c,)

    def _update_batch(self, plan: Plan, arena: Arena, ub: dict, consts: dict, b: int, stream: int) -> None:
        lib = _lib.load()
        up = plan.update
        base, end = arena.bases[b], arena.ends[b]

        def col(name: str) -> int:
            t = arena.cols[name]
            return t.data_ptr() + base * t.element_size()

        d = _lib.plx_update_desc()
        d.n = end - base
        d.rule = up.rule_code
        d.src = col("from_id")
        d.dst = col("to_id")
        d.weight = col("weight")
        for k, name in enumerate(up.state_columns()):
            setattr(d, f"s{k}", col(name))
        d.gfield = ub[up.grad_field.name].data_ptr()
        d.act = ub[ACTIVATION.name].data_ptr()
        if "pow_table" in consts:
            d.pow_table = consts["pow_table"].data_ptr()
            d.pow_table_len = consts["pow_table"].numel() // 2
        for k, v in enumerate(up.params()):
            d.p[k] = float(v)
        self._edge_state(d, arena, b, True)
        d.live_end -= base
        d.dead = col("dead") if arena.dead_in_rows else None
        t, keep = self._update_tiles(arena, b)
        self._launch("update_conn", lib.plx_update_batch_tiles, d, t, self.batch, stream)
        del keep
        self._advance_t(arena, b)


def make_batched_step(plan: Plan, static: NetworkStatic, batch_size: int) -> Any:
    return BatchedStepFn(plan, static, batch_size)
