"""Host driver: runs the step loop and owns the structural recoveries
(src/plastax/driver.py:1-420).

After every step the driver reads the state's flags. An overflowing growth
is completed inside the same step: every full bucket grows (``grow_bucket``)
and the candidates the claim dropped claim the new room (the growth phase's
retry), in the total order, until none is left -- exactly what the step would
have committed had the buckets been that large from the start. Then, when
``needs_resort`` is raised, a TOPOLOGICAL network is resorted (levels
recomputed from the live edges, buckets laid out again); a PIPELINE network
never resorts. With ``check_every = N > 1`` the flags are read every N
steps: an overflow grows every bucket with fewer free slots than the growth
rule's ``max_new_per_level`` (the dropped candidates are not grown) and a
resort waits for the check.

The step and the structural phases run on the GPU; the driver's decisions
read a few scalars back to the host, as the reference's do.
"""

from __future__ import annotations

from typing import Any, Callable

import numpy as np
import torch

from plastax_amd._types import Propagation
from plastax_amd.state import NetworkState, NetworkStatic, grow_bucket
from plastax_amd.step import StepFn, StepInputs, StepResult, make_step


def _loss_record(result: StepResult) -> Any:
    return result.loss


class Driver:
    """Runs a network's step loop, owning regrow-and-retry and resort
    (driver.py:67-392)."""

    def __init__(self, net: type, static: NetworkStatic, state: NetworkState, *, check_every: int = 1,
                 batch_size: int | None = None, layout: str = "auto", fuse_prune: str = "auto",
                 growth: str = "auto") -> None:
        if check_every < 1:
            raise ValueError(f"Driver: check_every must be >= 1, got {check_every}")
        self._net = net
        self._static = static
        self._state = state
        self._kw = dict(batch_size=batch_size, layout=layout, fuse_prune=fuse_prune, growth=growth)
        self._resorts = net.propagation is Propagation.TOPOLOGICAL
        self._step: StepFn = self._make_step()
        self._check_every = check_every
        self._since_check = 0
        self._overflowed = False
        self.regrows = 0
        self.resorts = 0
        self._graphs: dict = {}  # scan's captured chunks

    @property
    def state(self) -> NetworkState:
        return self._state

    @property
    def static(self) -> NetworkStatic:
        return self._static

    def _make_step(self) -> StepFn:
        return make_step(self._net, self._static, **self._kw)

    # -- the loop ---------------------------------------------------------------
    def step(self, inputs: StepInputs) -> StepResult:
        """One step; an overflowing growth is completed and a due resort run
        before returning (driver.py:134-168)."""
        if self._check_every > 1:
            return self._deferred_step(inputs)
        result = self._step(self._state, inputs)
        state = self._complete_growth(result.state)
        self._state = self._resort_if_due(state)
        return StepResult(state=self._state, overflow=self._state.overflow, loss=result.loss)

    def scan(self, inputs: StepInputs, *, record: Callable[[StepResult], Any] | None = None,
             steps: int | None = None, graph: bool | None = None) -> Any:
        """Run a chunk of steps (inputs and targets with a leading chunk axis)
        with `step`'s semantics; returns the per-step records stacked along
        a leading axis (the loss by default), entries at or beyond ``steps``
        zero (driver.py:170-270).

        The reference runs the chunk as one device-side loop. Here, for a
        streaming step without structural phases or reset_global (nothing
        the host must decide between steps), the chunk's first step runs as
        usual and the other steps are captured once into a HIP graph and
        replayed -- one launch for the chunk, no dispatch per step -- with
        the inputs copied into the graph's buffers; the results are step for
        step those of `step`. ``graph``: None uses the graph where it
        applies and ``record`` is the default; True requires it (``record``
        must then return device tensors); False runs the steps one by one.
        """
        rec = _loss_record if record is None else record
        xs = inputs.inputs
        if getattr(xs, "ndim", 0) < 2:
            raise ValueError(f"Driver.scan: inputs need a leading chunk axis, got shape {tuple(xs.shape)}")
        length = int(xs.shape[0])
        if inputs.targets is not None and int(inputs.targets.shape[0]) != length:
            raise ValueError("Driver.scan: targets chunk axis does not match the inputs'")
        count = length if steps is None else int(steps)
        if not 0 <= count <= length:
            raise ValueError(f"Driver.scan: steps must be in [0, {length}], got {steps}")
        why = self._graph_refusal()
        if graph is True and why:
            raise ValueError(f"Driver.scan(graph=True): {why}")
        if count >= 2 and not why and (graph is True or (graph is None and record is None)):
            return self._scan_graph(inputs, rec, count, length)
        out = []
        for i in range(count):
            t = None if inputs.targets is None else inputs.targets[i]
            out.append(rec(self.step(StepInputs(xs[i], t))))
        if not out:
            return np.zeros((length,), np.float32)
        first = out[0]
        if isinstance(first, torch.Tensor):
            pad = [torch.zeros_like(first)] * (length - count)
            return torch.stack([o.reshape(first.shape) for o in out] + pad)
        return np.concatenate([np.asarray(out), np.zeros((length - count,) + np.shape(first))])

    def _graph_refusal(self) -> str:
        """Why a chunk cannot run as a captured graph ('' when it can)."""
        step = self._step
        if not isinstance(step, StepFn) or self._kw.get("batch_size") is not None:
            return "batched steps run step by step"
        if self._check_every != 1:
            return "check_every > 1 reads flags between steps"
        plan = step.plan
        if plan.prune_unit or plan.prune_conn or plan.add_unit or plan.add_conn is not None:
            return "structural phases decide on the host between steps"
        if plan.reset_global:
            return "reset_global changes the globals on the host every step"
        if plan.forward.generic is not None or (plan.backward is not None and plan.backward.generic is not None):
            return "generic passes run step by step"
        if self._state.device.type != "cuda":
            return "the state is not on a GPU"
        return ""

    def _scan_graph(self, inputs: StepInputs, rec: Callable[[StepResult], Any], count: int, length: int) -> Any:
        """The chunk's first step eagerly (every first-use build and host
        read happens there), then steps 1.. as one replay of a captured
        graph (captured on first use for this arena, buffers and shapes)."""
        dev = self._state.device
        xs = torch.as_tensor(inputs.inputs, dtype=torch.float32, device=dev)
        ts = None if inputs.targets is None else torch.as_tensor(inputs.targets, dtype=torch.float32, device=dev)
        first = rec(self.step(StepInputs(xs[0], None if ts is None else ts[0])))
        state = self._state
        arena = self._step.arena(state)
        n = count - 1
        key = (n, rec, id(self._step), id(arena), tuple(xs.shape[1:]), None if ts is None else tuple(ts.shape[1:]),
               tuple(state._units), _globals_key(state.globals_))
        entry = self._graphs.get(key)
        if entry is not None:
            # The graph reads and writes the unit buffers it was captured on;
            # an eager PIPELINE step since then left the values in copies.
            for name, col in entry[4].items():
                if state._units[name] is not col:
                    col.copy_(state._units[name])
                    state._units[name] = col
        if entry is None:
            self._graphs.clear()  # one captured chunk at a time: its buffers stay allocated
            arena.drop_uniform_t()
            xin = torch.empty((n,) + tuple(xs.shape[1:]), dtype=torch.float32, device=dev)
            tin = None if ts is None else torch.empty((n,) + tuple(ts.shape[1:]), dtype=torch.float32, device=dev)
            xin.copy_(xs[1:count])
            if tin is not None:
                tin.copy_(ts[1:count])
            units = state._units
            orig = dict(units)
            g = torch.cuda.CUDAGraph()
            torch.cuda.synchronize(dev)
            with torch.cuda.graph(g):
                recs = []
                for i in range(n):
                    res = self._step(state, StepInputs(xin[i], None if tin is None else tin[i]))
                    state = res.state
                    recs.append(rec(res))
                out = torch.stack(recs)
                # Swapped unit buffers (a PIPELINE apply writes copies) go back
                # into the state's own, so every replay starts from them.
                for name, col in orig.items():
                    if state._units[name] is not col:
                        col.copy_(state._units[name])
            for name, col in orig.items():
                state._units[name] = col
            self._state = state
            entry = self._graphs[key] = (g, xin, tin, out, orig)
            g.replay()
        else:
            g, xin, tin, out, _ = entry
            xin.copy_(xs[1:count])
            if tin is not None:
                tin.copy_(ts[1:count])
            g.replay()
            state.step = int(state.step) + n
        result = torch.cat([torch.as_tensor(first, device=dev).reshape((1,) + tuple(out.shape[1:])), out.clone()])
        if count < length:
            pad = torch.zeros((length - count,) + tuple(result.shape[1:]), dtype=result.dtype, device=dev)
            result = torch.cat([result, pad])
        return result

    # -- recoveries ---------------------------------------------------------------
    def _free_slots(self, state: NetworkState, level: int) -> int:
        """Slots any level can still claim in bucket `level` (driver.py:373-382)."""
        cap = int(self._static.level_capacities[level])
        if self._static.propagation is Propagation.PIPELINE:
            return cap - int(state.tail_start)
        return cap - int((state.conns[level]["dead"] == 0).sum())

    def _complete_growth(self, state: NetworkState) -> NetworkState:
        """Regrow every full bucket and let the dropped winners claim the new
        room, until none is left (driver.py:319-331)."""
        from plastax_amd import grow

        phase = self._step._grow
        while bool(state.overflow):
            for level in range(len(self._static.level_capacities)):
                if self._free_slots(state, level) == 0:
                    self._static, state = grow_bucket(self._static, state, level)
                    self.regrows += 1
            self._step = self._make_step()
            k = grow.Kernels(state.device, int(torch.cuda.current_stream(state.device).cuda_stream))
            out = phase.retry(k, state.units, state.conns, tail_start=int(state.tail_start))
            state.conns = out.conns
            state.grown = int(state.grown) + out.grown
            state.overflow = out.overflow
            state.needs_resort = bool(state.needs_resort) or out.needs_resort
            state.tail_start = out.tail_start
        return state

    def _resort_if_due(self, state: NetworkState) -> NetworkState:
        """Resort a TOPOLOGICAL network whose flag is raised; PIPELINE never
        (driver.py:333-338)."""
        from plastax_amd.resort import resort

        if self._resorts and bool(state.needs_resort):
            self._static, state = resort(self._static, state)
            self._step = self._make_step()
            self.resorts += 1
        return state

    def _deferred_step(self, inputs: StepInputs) -> StepResult:
        """A `check_every > 1` step (driver.py:340-360)."""
        result = self._step(self._state, inputs)
        self._state = result.state
        self._overflowed = self._overflowed or bool(result.state.overflow)
        self._since_check += 1
        if self._since_check >= self._check_every:
            self._since_check = 0
            if self._overflowed:
                self._overflowed = False
                ac = self._net.add_conn
                want = (getattr(ac, "max_new_per_level", None) or 1) if ac is not None else 1
                state = self._state
                for level in range(len(self._static.level_capacities)):
                    if self._free_slots(state, level) < want:
                        self._static, state = grow_bucket(self._static, state, level)
                        self.regrows += 1
                self._state = state
                self._step = self._make_step()
            self._state = self._resort_if_due(self._state)
        return StepResult(state=self._state, overflow=self._state.overflow, loss=result.loss)


def _globals_key(g: Any) -> Any:
    """The globals' values (they are traced into the captured programs)."""
    if g is None:
        return None
    items = g.items() if isinstance(g, dict) else vars(g).items()
    return tuple(sorted((str(k), np.asarray(v).tobytes()) for k, v in items))
