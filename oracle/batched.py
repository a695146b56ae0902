"""CPU restatement of the reference's batched step -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, as the checker. It follows src/plastax/step.py:359-468 and
phases.py:217-532 over host arrays, per sample with `OracleNet`'s streaming
phases (forward in slot order per destination, the reference's literal
slot-order backward: `tile=None`), then once per batch:

- the exact connection update (phases.py:434-483): per edge
  ``total = stat_0; total = total + stat_b`` for b = 1 .. B-1 with
  ``stat_b = grad_field_b[dst] * activation_b[src]``, ``mean = total / B``,
  and the optimizer rule applied with that mean (the oracle's C rules, fed
  the per-edge mean through identity endpoints and a unit activation, so
  ``mean * 1.0`` is the gradient bit for bit);
- reduce_batch_units (phases.py:298-332): MEAN = samples summed in order
  from sample 0, then divided by B; SUM the same sum; FIRST sample 0; columns
  no per-sample phase writes keep their value;
- the structural phases and reset_global on the reduced state;
- the loss: ``(0 + l_0 + ... + l_{B-1}) / B``.

Parity pins: the reference's own batched assertions (a batch of one is the
streaming step; batched SGD is the mean of per-sample SGD steps; structural
phases run once per batch, tests/test_batched.py:117-230) and a float64
dense-matrix restatement of a batched MLP step (tests/test_batched_oracle.py).
"""

from __future__ import annotations

from typing import Any

import numpy as np

from oracle import oracle as ox


def written_columns(plan: Any, update_unit: list[str] = (), forward_generic: list[str] = (),
                    backward_generic: list[str] = ()) -> dict[str, str]:
    """The unit columns the per-sample phases write (phases.py:334-387);
    ``update_unit`` names the columns the traced update_unit writes,
    ``forward_generic`` / ``backward_generic`` those a generic pass's apply
    writes."""
    written = {"activation": "the input scatter"}
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


def reduce_column(red: str, cols: list[np.ndarray], batch: int) -> np.ndarray:
    """One column's batch reduction (phases.py:319-331)."""
    if red == "first":
        return cols[0].copy()
    s = cols[0].copy()
    for c in cols[1:]:
        s = (s + c).astype(cols[0].dtype)
    if red == "mean":
        s = (s / np.float32(batch)).astype(np.float32)
    return s


class OracleBatch:
    """A batched step over an `OracleNet`'s host arrays."""

    def __init__(self, net: "ox.OracleNet", batch: int) -> None:
        self.o = net
        self.batch = int(batch)
        net.tile = None  # the reference's slot-order backward, per sample

    def _update(self, per: list[dict[str, np.ndarray]]) -> None:
        o = self.o
        up = o.plan.update
        p = [float(v) for v in up.params()]
        B = self.batch
        gname = up.grad_field.name
        for c in o.conns:
            cap = c["dead"].size
            src, dst = c["from_id"].astype(np.int64), c["to_id"].astype(np.int64)
            live = ~c["dead"].astype(bool)
            s = np.clip(src, 0, o.static.num_units - 1)
            t = np.clip(dst, 0, o.static.num_units - 1)
            total = (per[0][gname][t] * per[0]["activation"][s]).astype(np.float32)
            for b in range(1, B):
                total = (total + (per[b][gname][t] * per[b]["activation"][s]).astype(np.float32)).astype(np.float32)
            mean = np.ascontiguousarray(np.where(live, total / np.float32(B), np.float32(0.0)).astype(np.float32))
            ones = np.ones(cap, dtype=np.float32)
            ar = np.arange(cap, dtype=np.int32)
            base = (cap, ox.iptr(ar), ox.iptr(ar), ox.bptr(c["dead"]), ox.fptr(c["weight"]))
            cols = [ox.fptr(c[name]) for name in up.state_columns()]
            lib = o.lib
            if up.rule_code == 0:
                lib.ox_update_sgd(*base, ox.fptr(mean), ox.fptr(ones), p[0])
            elif up.rule_code == 1:
                lib.ox_update_momentum(*base, *cols, ox.fptr(mean), ox.fptr(ones), p[0], p[1])
            elif up.rule_code == 2:
                lib.ox_update_adam(*base, *cols, ox.fptr(mean), ox.fptr(ones), *p[:7])
            else:
                lib.ox_update_rmsprop(*base, *cols, ox.fptr(mean), ox.fptr(ones), p[0], p[1], p[2], p[3])

    def _mean_of_writes(self, per: list[dict[str, np.ndarray]]) -> None:
        """A user UpdateConn under a batched step (phases.py:484-533): per
        sample, incoming then outgoing against the unchanged connections;
        every float32 column (written or not) takes old + (sum of the
        per-sample changes, in sample order) / B, a non-float written column
        sample 0's write."""
        from oracle import growth as og
        from plastax_amd import _site

        o = self.o
        B = self.batch
        if getattr(o, "_ucp", None) is None:
            udt = {s.name: np.dtype(s.dtype) for s in o.static.unit_fields}
            uc = o.plan.net.update_conn
            o._ucp = [_site.trace_conn_update(getattr(uc, d), d, udt, o.static.conn_fields, o.globals_)
                      for d in ("incoming", "outgoing")]
        old = o.conns
        totals = None
        first = None
        for b in range(B):
            new = og.update_conn(o._ucp, per[b], old, o.globals_)
            deltas = [{k: (nb[k] - ob[k]).astype(np.float32) for k in ob if ob[k].dtype == np.float32}
                      for nb, ob in zip(new, old)]
            if b == 0:
                totals, first = deltas, new
            else:
                totals = [{k: (t[k] + d[k]).astype(np.float32) for k in t} for t, d in zip(totals, deltas)]
        out = []
        for ob, nb0, tot in zip(old, first, totals):
            bucket = dict(ob)
            for k, v in ob.items():
                if v.dtype == np.float32:
                    bucket[k] = np.ascontiguousarray((v + tot[k] / np.float32(B)).astype(np.float32))
                else:
                    bucket[k] = np.ascontiguousarray(nb0[k])
            out.append(bucket)
        o.conns = out

    def step(self, inputs: Any, targets: Any = None) -> np.float32:
        """One batched step (step.py:402-468); returns the batch-mean loss."""
        o = self.o
        plan = o.plan
        B = self.batch
        x = np.asarray(inputs, dtype=np.float32).reshape(B, -1)
        tg = None if targets is None else np.asarray(targets, dtype=np.float32).reshape(B, -1)
        ids = np.asarray(o.static.input_ids, dtype=np.int64)
        shared = o.units
        per: list[dict[str, np.ndarray]] = []
        losses = np.zeros(B, dtype=np.float32)
        for b in range(B):
            o.units = {k: v.copy() for k, v in shared.items()}
            if ids.size:
                o.units["activation"][ids] = x[b]
            o.forward()
            if plan.loss is not None:
                losses[b] = np.float32(np.float32(0.0) + o.loss(tg[b]))
            if plan.backward is not None:
                o.backward()
            if getattr(plan, "update_unit", False):
                o.update_unit()
            per.append(o.units)
        o.units = shared
        if plan.update is not None:
            self._update(per)
        if getattr(plan, "update_generic", False):
            self._mean_of_writes(per)
        policy = plan.net.batch_reduction
        specs = {s.name: s for s in o.static.unit_fields}
        reduced = dict(shared)
        uu = list(getattr(o, "_uu", (None, []))[1]) if getattr(plan, "update_unit", False) else []
        gen = [list(o._gen(w)[3]) if pp is not None and pp.generic is not None else []
               for w, pp in (("fwd", plan.forward), ("bwd", plan.backward))]
        for name in written_columns(plan, uu, *gen):
            red = policy.reduction(specs[name])
            reduced[name] = np.ascontiguousarray(reduce_column(red.value, [u[name] for u in per], B))
        o.units = reduced
        if (getattr(plan, "prune_unit", False) or getattr(plan, "prune_conn", False)
                or getattr(plan, "add_unit", False) or getattr(plan, "add_conn", None) is not None):
            o.structural()
        if getattr(plan, "reset_global", False):
            o.globals_ = plan.net.reset_global.reset(o.globals_)
        o.step_count += 1
        s = np.float32(0.0)
        for b in range(B):
            s = np.float32(s + losses[b])
        return np.float32(s / np.float32(B))
