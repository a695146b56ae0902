"""CPU oracle of the streaming step -- TEST INFRASTRUCTURE ONLY.

Restates the reference's step (src/plastax/step.py:578-618 and the phase
builders of src/plastax/phases.py) over the *logical* arena, i.e. the
reference's own layout: per-bucket dicts of columns in slot order. The O(E)
loops run in plastax_oracle.c (built by the Makefile beside this file); the
level walks below follow phases.py line by line:

- forward, TOPOLOGICAL: phases.py:972-1015 (accumulate bucket l, finalize
  level l+1, non-input, live); PIPELINE: sweep.py:287-340 (one sweep,
  every non-input unit);
- loss: phases.py:1107-1131 (seed written at the output ids);
- backward, TOPOLOGICAL: phases.py:1049-1104 (prime the deepest level from
  the identity, then buckets L-1..1; bucket 0 is never reduced); PIPELINE:
  sweep.py:402-449 (every unit, inputs included);
- update_conn: phases.py:1196-1242 with the optim rules.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
this module, as the checker. The policies' apply / loss programs are the
ones the framework traced (plastax_amd._expr); this file evaluates them with
its own interpreter.
"""

from __future__ import annotations

import ctypes
import pathlib
import subprocess
from typing import Any

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libplastax_oracle.so"
PIECE = 256  # loss folds: pieces of 256 outputs
TILE = 4096  # backward folds: tiles of at most this many positions
NSUPER = 512  # backward folds: superblocks per bucket at most

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_lib: ctypes.CDLL | None = None


def tiles_of_positions(span: int, tile: int, nsuper_max: int) -> tuple[np.ndarray, np.ndarray]:
    """Tile and superblock of every position of a bucket span (the device's
    fold structure): min(nsuper_max, ceil(span/tile)) superblocks, the k-th
    starting at floor(k*span/nsuper) rounded down to a multiple of 4, each
    cut into tiles of `tile` positions from its start. Returns per-position
    (global tile index, superblock index)."""
    if span == 0:
        return np.zeros(0, np.int32), np.zeros(0, np.int32)
    nsuper = min(nsuper_max, -(-span // tile))
    k = np.arange(nsuper + 1, dtype=np.int64)
    starts = (k * span // nsuper) & ~3
    starts[-1] = span
    pos = np.arange(span, dtype=np.int64)
    sb = np.searchsorted(starts, pos, side="right") - 1
    tiles_per_sb = -(-(starts[1:] - starts[:-1]) // tile)
    first_tile = np.concatenate([[0], np.cumsum(tiles_per_sb)])
    tile_ix = first_tile[sb] + (pos - starts[sb]) // tile
    return tile_ix.astype(np.int32), sb.astype(np.int32)


def physical_unit_index(levels: np.ndarray, conns: list[dict[str, np.ndarray]]) -> np.ndarray:
    """The device's unit numbering, restated: units ordered by level, then by
    live out-degree descending, then by id. Returns, for every unit id, its
    physical index (the device's destination-sorted order sorts by it)."""
    n = levels.size
    outdeg = np.zeros(n, dtype=np.int64)
    for c in conns:
        live = ~c["dead"].astype(bool)
        outdeg += np.bincount(c["from_id"][live].astype(np.int64), minlength=n)
    order = sorted(range(n), key=lambda u: (int(levels[u]), -int(outdeg[u]), u))
    index = np.empty(n, dtype=np.int64)
    index[np.asarray(order, dtype=np.int64)] = np.arange(n)
    return index


def build() -> pathlib.Path:
    """Compile the C restatement (make)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def load() -> ctypes.CDLL:
    """The C restatement (built on first use), its signatures declared."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = _declare(ctypes.CDLL(str(LIB_PATH)))
    return _lib


def load_variant(path: pathlib.Path) -> ctypes.CDLL:
    """Another build of the same source (e.g. the perturbation build),
    its signatures declared; not cached."""
    if not path.exists():
        build()
    return _declare(ctypes.CDLL(str(path)))


def _declare(lib: ctypes.CDLL) -> ctypes.CDLL:
    for name in ("ox_expf", "ox_logf", "ox_tanhf", "ox_sigmoidf", "ox_cosf", "ox_sinf", "ox_log1pf", "ox_expm1f"):
        getattr(lib, name).restype = ctypes.c_float
        getattr(lib, name).argtypes = [ctypes.c_float]
    lib.ox_pow_step.restype = ctypes.c_float
    lib.ox_pow_step.argtypes = [ctypes.c_float, ctypes.c_float]
    lib.ox_philox32.restype = ctypes.c_uint32
    lib.ox_philox32.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
    lib.ox_philox4x32_10.argtypes = [ctypes.POINTER(ctypes.c_uint32)] * 3
    lib.ox_site_seed.restype = ctypes.c_uint64
    lib.ox_site_seed.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
    lib.ox_conn_key.restype = ctypes.c_uint32
    lib.ox_conn_key.argtypes = [ctypes.c_uint32] * 3
    lib.ox_site_draw.restype = ctypes.c_uint32
    lib.ox_site_draw.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32]
    lib.ox_uniform_int.restype = ctypes.c_uint32
    lib.ox_uniform_int.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
    lib.ox_unit_float.restype = ctypes.c_float
    lib.ox_unit_float.argtypes = [ctypes.c_uint32]
    lib.ox_loss_elementwise.restype = ctypes.c_float
    lib.ox_loss_softmax_ce.restype = ctypes.c_float
    lib.ox_identity.restype = ctypes.c_float
    lib.ox_identity.argtypes = [ctypes.c_int32]
    lib.ox_bucket_reduce_fwd.argtypes = [
        ctypes.c_int64, _i32p, _i32p, _u8p, _f32p, _f32p, ctypes.c_int32, _f32p
    ]
    lib.ox_bucket_reduce_bwd.argtypes = [
        ctypes.c_int64, _i32p, _i32p, _u8p, _f32p, _f32p, ctypes.c_int32,
        ctypes.c_int32, ctypes.c_int32, _f32p, _f32p, _i32p,
    ]
    lib.ox_bucket_reduce_bwd_tiled.argtypes = [
        ctypes.c_int64, ctypes.POINTER(ctypes.c_int64), _i32p, _i32p, _f32p, _f32p,
        _i32p, _i32p, ctypes.c_int32, _f32p,
    ]
    lib.ox_combine.argtypes = [ctypes.c_int64, ctypes.c_int32, _f32p, _f32p]
    _i64p = ctypes.POINTER(ctypes.c_int64)
    lib.ox_bucket_reduce_fwd_rows.argtypes = [
        ctypes.c_int64, _i64p, _i64p, _i32p, _i32p, _f32p, _f32p, ctypes.c_int32, _f32p,
    ]
    lib.ox_bucket_reduce_bwd_tiled_runs.argtypes = [
        ctypes.c_int64, _i64p, _i64p, _i32p, _i32p, _f32p, _f32p, _i32p, _i32p, ctypes.c_int32, _f32p,
    ]
    lib.ox_set_threads.restype = ctypes.c_int32
    lib.ox_set_threads.argtypes = [ctypes.c_int32]
    lib.ox_apply.argtypes = [
        _i32p, ctypes.c_int32, _f32p, ctypes.POINTER(_f32p), _i32p, ctypes.c_int32,
        ctypes.c_int64, _f32p, _u8p, ctypes.c_int32, _f32p,
    ]
    lib.ox_loss_elementwise.argtypes = [
        _i32p, ctypes.c_int32, _f32p, ctypes.POINTER(_f32p), _i32p, ctypes.c_int32,
        _f32p, _f32p, _f32p, ctypes.c_int32,
    ]
    lib.ox_loss_softmax_ce.argtypes = [
        _f32p, _i32p, ctypes.c_int32, _f32p, _f32p, _f32p, ctypes.c_int32
    ]
    upd = [ctypes.c_int64, _i32p, _i32p, _u8p, _f32p]
    lib.ox_update_sgd.argtypes = upd + [_f32p, _f32p, ctypes.c_float]
    lib.ox_update_momentum.argtypes = upd + [_f32p, _f32p, _f32p, ctypes.c_float, ctypes.c_float]
    lib.ox_update_adam.argtypes = upd + [_f32p, _f32p, _f32p, _f32p, _f32p] + [ctypes.c_float] * 7
    lib.ox_update_rmsprop.argtypes = upd + [_f32p, _f32p, _f32p] + [ctypes.c_float] * 4
    lib.ox_free_block_counts.argtypes = [ctypes.c_int64, _u8p, ctypes.c_int32, _i32p]
    lib.ox_nth_free_slots.restype = ctypes.c_int64
    lib.ox_nth_free_slots.argtypes = [
        ctypes.c_int64, _u8p, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)
    ]
    return lib



def ptr(a: np.ndarray, ctype: Any) -> Any:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def fptr(a: np.ndarray) -> Any:
    assert a.dtype == np.float32
    return ptr(a, ctypes.c_float)


def iptr(a: np.ndarray) -> Any:
    assert a.dtype == np.int32
    return ptr(a, ctypes.c_int32)


def bptr(a: np.ndarray) -> Any:
    assert a.dtype in (np.uint8, np.bool_)
    return ptr(a.view(np.uint8), ctypes.c_uint8)


class _ProgramArgs:
    """A traced program's code/consts and its field-pointer table."""

    def __init__(self, prog: Any, units: dict[str, np.ndarray], globals_: Any) -> None:
        self.code = np.ascontiguousarray(prog.flat_code(), dtype=np.int32)
        self.consts = np.ascontiguousarray(prog.const_values(globals_), dtype=np.float32)
        if self.consts.size == 0:
            self.consts = np.zeros(1, np.float32)
        names = list(prog.fields)
        fixed = dict(getattr(prog, "fixed_at", {}))
        # A field read at one fixed unit (a loss's u[F, UnitIdx(k)]) is handed
        # over as a column holding that unit's value at every index.
        cols = [np.full(units[n].shape, units[n][fixed[k]], dtype=units[n].dtype) if k in fixed else units[n]
                for k, n in enumerate(names)]
        out_idx = []
        for name in prog.out_fields:
            if name is None:
                out_idx.append(-1)
                continue
            own = [k for k, n in enumerate(names) if n == name and k not in fixed]
            if not own:
                names.append(name)
                cols.append(units[name])
                own = [len(names) - 1]
            out_idx.append(own[0])
        self.names = names
        self._cols = cols  # kept alive: the table points into them
        self.table = (_f32p * max(len(names), 1))(*[fptr(c) for c in cols])
        self.out_idx = np.asarray(out_idx, dtype=np.int32)
        self.ninstr = prog.ninstr


class OracleNet:
    """The reference step over host copies of a logical arena."""

    def __init__(
        self,
        static: Any,
        units: dict[str, np.ndarray],
        conns: list[dict[str, np.ndarray]],
        plan: Any,
        globals_: Any = None,
        *,
        piece: int = PIECE,
        tile: int | None = TILE,
        nsuper: int = NSUPER,
        parallel: bool = False,
    ) -> None:
        self.static = static
        # parallel: the forward folds by destination rows and the tiled
        # backward by source runs (the same folds, so the same bits), which
        # lets the C loops run on the OpenMP team (ox_set_threads).
        self.parallel = parallel
        self._fwd_rows: dict = {}
        self.units = {k: np.ascontiguousarray(v) for k, v in units.items()}
        self.conns = [{k: np.ascontiguousarray(v) for k, v in b.items()} for b in conns]
        self.plan = plan
        self.globals_ = globals_
        self.piece = piece
        self.tile = tile
        self.nsuper = nsuper
        self._bwd_order: dict[int, tuple[np.ndarray, np.ndarray, np.ndarray]] = {}
        self._phys_index: np.ndarray | None = None
        self.step_count = 0
        # Structural state (phases.py:4490-5203) and the traced predicate.
        self.tail_start = 0
        self.needs_resort = False
        self.grown = 0
        self.overflow = False
        self.units_added = 0
        self.unit_overflow = False
        self.remainder: Any = None
        self._prune_prog: Any = None
        n = static.num_units
        self.is_input = np.zeros(n, dtype=bool)
        if static.input_ids:
            self.is_input[np.asarray(static.input_ids)] = True
        self.pipeline = static.propagation.value == "pipeline"
        self.lib = load()

    # -- helpers ------------------------------------------------------------
    def _live(self) -> np.ndarray:
        pruned = self.units.get("pruned")
        n = self.static.num_units
        return np.ones(n, dtype=bool) if pruned is None else ~pruned.astype(bool)

    def _apply(self, pp: Any, acc: np.ndarray, mask: np.ndarray) -> None:
        lib = self.lib
        n = self.static.num_units
        args = _ProgramArgs(pp.program, self.units, self.globals_)
        nout = len(pp.program.out_fields)
        scratch = np.zeros(max(nout, 1) * n, dtype=np.float32)
        m = np.ascontiguousarray(mask.astype(np.uint8))
        lib.ox_apply(
            iptr(args.code), args.ninstr, fptr(args.consts), args.table, iptr(args.out_idx),
            nout, n, fptr(acc), bptr(m), pp.monoid, fptr(scratch),
        )

    def _rows(self, b: int) -> tuple[np.ndarray, ...]:
        """(row_ptr, row_slots, row_unit) of bucket b: its live slots
        grouped by destination, ascending slot order inside a destination.
        Cached with the structure (the structural phases drop the cache)."""
        hit = self._fwd_rows.get(b)
        if hit is not None:
            return hit
        c = self.conns[b]
        live = np.flatnonzero(~c["dead"].astype(bool))
        slots = live[np.argsort(c["to_id"][live], kind="stable")].astype(np.int64)
        dst = c["to_id"][slots]
        if slots.size == 0:  # no live edge: no row
            starts = np.zeros(1, dtype=np.int64)
        else:
            starts = np.concatenate([[0], np.flatnonzero(np.diff(dst)) + 1, [slots.size]]).astype(np.int64)
        units = np.ascontiguousarray(dst[starts[:-1]].astype(np.int32))
        self._fwd_rows[b] = (starts, np.ascontiguousarray(slots), units)
        return self._fwd_rows[b]

    def _factors(self, b: int, pp: Any) -> tuple[np.ndarray, np.ndarray]:
        """(connection factor per slot, unit factor per unit) of a pass's
        product map: WEIGHT and the gathered field, or the map's constants
        spread over the bucket's slots / the units (the term is their float32
        product either way)."""
        c = self.conns[b]
        w = c["weight"] if pp.w_const is None else np.full(c["dead"].size, pp.w_const, np.float32)
        x = (self.units[pp.field] if pp.field is not None
             else np.full(self.static.num_units, pp.x_const, np.float32))
        return w, x

    def _reduce_fwd(self, b: int, pp: Any) -> np.ndarray:
        c = self.conns[b]
        n = self.static.num_units
        monoid = pp.monoid
        weight, x = self._factors(b, pp)
        out = np.full(n, self.lib.ox_identity(monoid), dtype=np.float32)
        if self.parallel:
            starts, slots, units = self._rows(b)
            self.lib.ox_bucket_reduce_fwd_rows(
                units.size, starts.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                slots.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), iptr(units),
                iptr(c["from_id"]), fptr(weight), fptr(x), monoid, fptr(out),
            )
            return out
        self.lib.ox_bucket_reduce_fwd(
            c["dead"].size, iptr(c["from_id"]), iptr(c["to_id"]), bptr(c["dead"]),
            fptr(weight), fptr(x), monoid, fptr(out),
        )
        return out

    def _tiles(self, b: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """(order, tile, sb) of bucket b's live slots: order sorts them by
        (src, physical dst, slot); a slot's physical position is its rank in
        (physical dst, slot) order, and tile / sb are that position's tile
        and superblock over the bucket's span (capacity rounded up to 4).
        Cached (the structure is static)."""
        if self._phys_index is None:
            self._phys_index = physical_unit_index(self.units["level"], self.conns)
        if b not in self._bwd_order:
            c = self.conns[b]
            cap = c["dead"].size
            live = np.flatnonzero(~c["dead"].astype(bool))
            dst = self._phys_index[c["to_id"][live]]
            src = c["from_id"][live]
            rank = np.empty(live.size, dtype=np.int64)
            rank[np.lexsort((live, dst))] = np.arange(live.size)
            tile = np.zeros(cap, dtype=np.int32)
            sb = np.zeros(cap, dtype=np.int32)
            if self.tile:
                t_pos, s_pos = tiles_of_positions(-(-cap // 4) * 4, self.tile, self.nsuper)
                tile[live] = t_pos[rank]
                sb[live] = s_pos[rank]
            order = np.ascontiguousarray(live[np.lexsort((live, dst, src))].astype(np.int64))
            self._bwd_order[b] = (order, tile, sb)
        return self._bwd_order[b]

    def _reduce_bwd(self, b: int, pp: Any) -> np.ndarray:
        c = self.conns[b]
        n = self.static.num_units
        monoid = pp.monoid
        weight, gx = self._factors(b, pp)
        out = np.full(n, self.lib.ox_identity(monoid), dtype=np.float32)
        if self.tile is None:
            # the reference's literal slot-order fold
            pc = np.zeros(n, dtype=np.float32)
            pn = np.zeros(n, dtype=np.int32)
            self.lib.ox_bucket_reduce_bwd(
                c["dead"].size, iptr(c["from_id"]), iptr(c["to_id"]), bptr(c["dead"]),
                fptr(weight), fptr(gx), n, monoid, 1 << 30,
                fptr(out), fptr(pc), iptr(pn),
            )
            return out
        order, tile, sb = self._tiles(b)
        # Edges tombstoned since the layout was fixed contribute the identity,
        # i.e. nothing: every fold starts from the identity.
        dead_now = c["dead"].astype(bool)[order]
        if dead_now.any():
            order = np.ascontiguousarray(order[~dead_now])
        if self.parallel:
            run_off = self._fwd_rows.get(("runs", b)) if not dead_now.any() else None
            if run_off is None:
                fr = c["from_id"][order]
                run_off = np.concatenate([[0], np.flatnonzero(np.diff(fr)) + 1, [order.size]]).astype(np.int64)
                if not dead_now.any():
                    self._fwd_rows[("runs", b)] = run_off
            self.lib.ox_bucket_reduce_bwd_tiled_runs(
                run_off.size - 1, run_off.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                order.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                iptr(c["from_id"]), iptr(c["to_id"]), fptr(weight),
                fptr(gx), iptr(tile), iptr(sb), monoid, fptr(out),
            )
            return out
        self.lib.ox_bucket_reduce_bwd_tiled(
            order.size, order.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
            iptr(c["from_id"]), iptr(c["to_id"]), fptr(weight),
            fptr(gx), iptr(tile), iptr(sb), monoid, fptr(out),
        )
        return out

    # -- phases ---------------------------------------------------------------
    # -- generic passes (plastax_amd/generic.py) -----------------------------
    def _gen(self, which: str) -> tuple:
        """(GenericPass, map program, apply program, apply's written fields)."""
        key = "_gen_" + which
        if getattr(self, key, None) is None:
            from plastax_amd import _site

            pp = self.plan.forward if which == "fwd" else self.plan.backward
            gp = pp.generic
            udt = {s.name: np.dtype(s.dtype) for s in self.static.unit_fields}
            cdt = {s.name: np.dtype(s.dtype) for s in self.static.conn_fields}
            mprog = _site.trace_pass_map(gp.policy, gp.backward, udt, cdt, self.globals_)
            aprog, names = _site.trace_pass_apply(gp.policy, len(gp.monoids), gp.tuple_acc, udt, self.globals_)
            setattr(self, key, (gp, mprog, aprog, names))
        return getattr(self, key)

    @staticmethod
    def _gen_op(m: int, a: Any, b: Any) -> Any:
        """A named monoid on float32 arrays, with the device's NaN and
        tie rules (max / min keep the first operand only when it compares
        strictly greater / less)."""
        a = np.asarray(a, dtype=np.float32)
        b = np.asarray(b, dtype=np.float32)
        if m == 0:
            return (a + b).astype(np.float32)
        if m == 1:
            return (a * b).astype(np.float32)
        pick = (a > b) if m == 2 else (a < b)
        return np.where(np.isnan(a), a, np.where(np.isnan(b), b, np.where(pick, a, b))).astype(np.float32)

    def _gen_reduce(self, which: str, b: int) -> list[np.ndarray]:
        """Per-unit folds of bucket b's live edges, each row's edges in slot
        order from the identity (rows: destinations forward, sources
        backward); the identity where a unit has none."""
        from oracle import growth as og

        gp, mprog, _, _ = self._gen(which)
        n = self.static.num_units
        c = self.conns[b]
        cap = c["dead"].size
        roles = {"cid": np.arange(cap, dtype=np.int32), "src": c["from_id"], "dst": c["to_id"]}
        terms = og.site_eval(mprog, cap, roles, self.units, self.globals_, conns=c)
        live = np.flatnonzero(~c["dead"].astype(bool))
        key = c["from_id"] if gp.backward else c["to_id"]
        order = live[np.argsort(key[live], kind="stable")]
        rows = key[order]
        outs = [np.full(n, v, dtype=np.float32) for v in gp.identities]
        bounds = np.concatenate([[0], np.flatnonzero(np.diff(rows)) + 1, [rows.size]]) if rows.size else [0]
        for lo, hi in zip(bounds[:-1], bounds[1:]):
            u = int(rows[lo])
            for k, (m, ident) in enumerate(zip(gp.monoids, gp.identities)):
                s = np.float32(ident)
                for v in terms[k][order[lo:hi]]:
                    s = self._gen_op(m, s, v)
                outs[k][u] = s
        return outs

    def _gen_apply(self, which: str, acc: list[np.ndarray], mask: np.ndarray) -> None:
        from oracle import growth as og
        from plastax_amd import _site

        gp, _, aprog, names = self._gen(which)
        fin = np.flatnonzero(mask).astype(np.int32)
        if fin.size and names:
            units = dict(self.units)
            units.update(dict(zip(_site.acc_field_names(len(acc)), acc)))
            vals = og.site_eval(aprog, fin.size, {"i": fin}, units, self.globals_)
            live = self._live()[fin]
            for name, v in zip(names, vals):
                col = self.units[name]
                col[fin[live]] = np.asarray(v, dtype=col.dtype)[live]
        for a, v in zip(acc, gp.identities):
            a[fin] = np.float32(v)

    def _gen_forward(self) -> None:
        gp = self.plan.forward.generic
        n = self.static.num_units
        levels = self.units["level"]
        live = np.ones(n, dtype=bool)  # pruned units are skipped by the apply's writes
        acc = [np.full(n, v, dtype=np.float32) for v in gp.identities]
        nb = len(self.conns)
        for lv in range(nb):
            out = self._gen_reduce("fwd", lv)
            acc = [self._gen_op(m, a, o) for m, a, o in zip(gp.monoids, acc, out)]
            if not self.pipeline:
                self._gen_apply("fwd", acc, (levels == lv + 1) & ~self.is_input & live)
        if self.pipeline:
            self._gen_apply("fwd", acc, ~self.is_input & live)

    def _gen_backward(self) -> None:
        gp = self.plan.backward.generic
        n = self.static.num_units
        levels = self.units["level"]
        acc = [np.full(n, v, dtype=np.float32) for v in gp.identities]
        nb = len(self.conns)
        if self.pipeline:
            out = self._gen_reduce("bwd", 0)
            acc = [self._gen_op(m, a, o) for m, a, o in zip(gp.monoids, acc, out)]
            self._gen_apply("bwd", acc, np.ones(n, dtype=bool))
            return
        self._gen_apply("bwd", acc, (levels == nb) & ~self.is_input)
        for lv in range(nb - 1, 0, -1):
            out = self._gen_reduce("bwd", lv)
            acc = [self._gen_op(m, a, o) for m, a, o in zip(gp.monoids, acc, out)]
            self._gen_apply("bwd", acc, (levels == lv) & ~self.is_input)

    def forward(self) -> None:
        fp = self.plan.forward
        if fp.generic is not None:
            self._gen_forward()
            return
        n = self.static.num_units
        levels = self.units["level"]
        live = self._live()
        acc = np.full(n, fp.identity, dtype=np.float32)
        nb = len(self.conns)
        if self.pipeline:
            self.lib.ox_combine(n, fp.monoid, fptr(acc), fptr(self._reduce_fwd(0, fp)))
            self._apply(fp, acc, ~self.is_input & live)
            return
        for lv in range(nb):
            out = self._reduce_fwd(lv, fp)
            self.lib.ox_combine(n, fp.monoid, fptr(acc), fptr(out))
            self._apply(fp, acc, (levels == lv + 1) & ~self.is_input & live)

    def loss(self, targets: np.ndarray) -> np.float32:
        lp = self.plan.loss
        out_ids = np.asarray(self.static.output_ids, dtype=np.int32)
        t = np.ascontiguousarray(np.asarray(targets, dtype=np.float32).reshape(-1))
        seed = np.zeros(out_ids.size, dtype=np.float32)
        terms = np.zeros(max(out_ids.size, 1), dtype=np.float32)
        if lp.kind == "softmax":
            val = self.lib.ox_loss_softmax_ce(
                fptr(self.units["activation"]), iptr(out_ids), out_ids.size, fptr(t),
                fptr(seed), fptr(terms), self.piece,
            )
        else:
            args = _ProgramArgs(lp.program, self.units, self.globals_)
            val = self.lib.ox_loss_elementwise(
                iptr(args.code), args.ninstr, fptr(args.consts), args.table, iptr(out_ids),
                out_ids.size, fptr(t), fptr(seed), fptr(terms), self.piece,
            )
        self.units[lp.seed_field][out_ids] = seed
        return np.float32(val)

    def backward(self) -> None:
        bp = self.plan.backward
        if bp.generic is not None:
            self._gen_backward()
            return
        n = self.static.num_units
        levels = self.units["level"]
        live = self._live()
        acc = np.full(n, bp.identity, dtype=np.float32)
        nb = len(self.conns)
        if self.pipeline:
            self.lib.ox_combine(n, bp.monoid, fptr(acc), fptr(self._reduce_bwd(0, bp)))
            self._apply(bp, acc, live)
            return
        self._apply(bp, acc, (levels == nb) & ~self.is_input & live)
        for lv in range(nb - 1, 0, -1):
            out = self._reduce_bwd(lv, bp)
            self.lib.ox_combine(n, bp.monoid, fptr(acc), fptr(out))
            self._apply(bp, acc, (levels == lv) & ~self.is_input & live)

    def update(self) -> None:
        if getattr(self.plan, "update_generic", False):
            from oracle import growth as og
            from plastax_amd import _site

            if getattr(self, "_ucp", None) is None:
                udt = {s.name: np.dtype(s.dtype) for s in self.static.unit_fields}
                uc = self.plan.net.update_conn
                self._ucp = [_site.trace_conn_update(getattr(uc, d), d, udt, self.static.conn_fields,
                                                     self.globals_) for d in ("incoming", "outgoing")]
            self.conns = og.update_conn(self._ucp, self.units, self.conns, self.globals_)
            return
        up = self.plan.update
        p = [float(v) for v in up.params()]
        g = self.units[up.grad_field.name]
        act = self.units["activation"]
        for c in self.conns:
            cap = c["dead"].size
            base = (cap, iptr(c["from_id"]), iptr(c["to_id"]), bptr(c["dead"]), fptr(c["weight"]))
            cols = [fptr(c[name]) for name in up.state_columns()]
            if up.rule_code == 0:
                self.lib.ox_update_sgd(*base, fptr(g), fptr(act), p[0])
            elif up.rule_code == 1:
                self.lib.ox_update_momentum(*base, *cols, fptr(g), fptr(act), p[0], p[1])
            elif up.rule_code == 2:
                self.lib.ox_update_adam(*base, *cols, fptr(g), fptr(act), *p[:7])
            else:
                self.lib.ox_update_rmsprop(*base, *cols, fptr(g), fptr(act), p[0], p[1], p[2], p[3])

    def step(self, inputs: Any, targets: Any = None) -> np.float32:
        """One streaming step (step.py:578-618); returns the loss."""
        ids = np.asarray(self.static.input_ids, dtype=np.int64)
        if ids.size:
            self.units["activation"][ids] = np.asarray(inputs, dtype=np.float32).reshape(-1)
        self.forward()
        loss = np.float32(0.0)
        if self.plan.loss is not None:
            loss = np.float32(np.float32(0.0) + self.loss(targets))
        if self.plan.backward is not None:
            self.backward()
        if getattr(self.plan, "update_unit", False):
            self.update_unit()
        if self.plan.update is not None or getattr(self.plan, "update_generic", False):
            self.update()
        if (getattr(self.plan, "prune_unit", False) or getattr(self.plan, "prune_conn", False)
                or getattr(self.plan, "add_unit", False) or getattr(self.plan, "add_conn", None) is not None):
            self.structural()
        if getattr(self.plan, "reset_global", False):
            self.globals_ = self.plan.net.reset_global.reset(self.globals_)
        self.step_count += 1
        return loss

    def _unit_dtypes(self) -> dict[str, np.dtype]:
        return {s.name: np.dtype(s.dtype) for s in self.static.unit_fields}

    def update_unit(self) -> None:
        """phases.py:1148-1193."""
        from oracle import growth as og
        from plastax_amd import _site

        if not hasattr(self, "_uu"):
            self._uu = _site.trace_update_unit(self.plan.net.update_unit, self._unit_dtypes(), self.globals_)
        self.units = og.update_unit(self._uu[0], self._uu[1], self.units, self.globals_)

    def structural(self) -> None:
        """prune_conn then add_conn (phases.py:87-182 order) on the logical
        arena. The backward's fold structure (tiles over the destination-
        sorted positions, unit renumbering) is the layout's: it is fixed when
        the arena is laid out and laid out again exactly when a growth phase
        fires, as the device does; tombstones set in between contribute the
        identity."""
        from oracle import growth as og
        from plastax_amd import _site

        net = self.plan.net
        unit_dtypes = {s.name: np.dtype(s.dtype) for s in self.static.unit_fields}
        conn_dtypes = {s.name: np.dtype(s.dtype) for s in self.static.conn_fields}
        if getattr(self.plan, "prune_unit", False):
            if not hasattr(self, "_pu"):
                self._pu = _site.trace_prune_unit(net.prune_unit, unit_dtypes, self.globals_)
            self.units, self.conns, _ = og.prune_unit(self._pu, self.static, self.units, self.conns, self.globals_)
            self._fwd_rows = {}  # (its incident kills: rows hold live slots only)
            self.units = {k: np.ascontiguousarray(v) for k, v in self.units.items()}
            self.conns = [{k: np.ascontiguousarray(v) for k, v in b.items()} for b in self.conns]
        if self.plan.prune_conn:
            if self._prune_prog is None:
                self._prune_prog = _site.trace_predicate(net.prune_conn, unit_dtypes, conn_dtypes, self.globals_)
            self.conns = og.prune_conn(self._prune_prog, self.units, self.conns, self.globals_)
            self._fwd_rows = {}  # the parallel forward's rows hold live slots only
        if getattr(self.plan, "add_unit", False):
            interval = int(getattr(net, "structural_interval", 1))
            if interval <= 1 or self.step_count % interval == 0:
                if not hasattr(self, "_au"):
                    spawn = _site.trace_spawn(net.add_unit, unit_dtypes, self.globals_)
                    init, names = _site.trace_unit_init(net.add_unit, unit_dtypes, self.globals_)
                    self._au = (spawn, init, names)
                self.units, self.units_added, self.unit_overflow, _ = og.add_unit(
                    *self._au, self.static, int(getattr(net, "max_levels", 1024)), self.units, self.globals_)
                if self.units_added:
                    # new units get rows when the arena is laid out again
                    self._bwd_order = {}
                    self._fwd_rows = {}
                    self._phys_index = None
            else:
                self.units_added, self.unit_overflow = 0, False
        if self.plan.add_conn is not None:
            res = og.add_conn(
                net, self.static, self.units, self.conns, step=self.step_count, globals_=self.globals_,
                tail_start=self.tail_start, units_added=self.units_added, needs_resort=self.needs_resort,
            )
            self.grown, self.overflow = res.grown, res.overflow
            self.remainder = res.remainder
            if res.fired:
                self.conns = [{k: np.ascontiguousarray(v) for k, v in b.items()} for b in res.conns]
                self.needs_resort = res.needs_resort
                self.tail_start = res.tail_start
                self._bwd_order = {}
                self._fwd_rows = {}
                self._phys_index = None


def free_block_counts(dead: np.ndarray, block: int) -> np.ndarray:
    """Per-block dead counts (phases.py:2595-2618)."""
    lib = load()
    d = np.ascontiguousarray(dead.astype(np.uint8))
    nb = -(-d.size // block)
    out = np.zeros(nb, dtype=np.int32)
    lib.ox_free_block_counts(d.size, bptr(d), block, iptr(out))
    return out


def nth_free_slots(dead: np.ndarray, n: int) -> np.ndarray:
    """The first n free slots in ascending slot order, -1 past the end
    (phases.py:2670-2754)."""
    lib = load()
    d = np.ascontiguousarray(dead.astype(np.uint8))
    out = np.zeros(n, dtype=np.int64)
    lib.ox_nth_free_slots(d.size, bptr(d), n, out.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)))
    return out


class OracleDriver:
    """The reference Driver's step loop (driver.py:134-168, :319-338) over
    an OracleNet: complete an overflowing growth (grow every full bucket,
    retry the dropped winners), then resort a TOPOLOGICAL net whose flag is
    raised. Every change of the arena's shape lays it out again."""

    def __init__(self, net: OracleNet) -> None:
        self.o = net

    def _relayout(self) -> None:
        self.o._bwd_order = {}
        self.o._fwd_rows = {}
        self.o._phys_index = None

    def _free(self, level: int) -> int:
        o = self.o
        cap = int(o.static.level_capacities[level])
        if o.pipeline:
            return cap - int(o.tail_start)
        return cap - int((~o.conns[level]["dead"].astype(bool)).sum())

    def step(self, inputs: Any, targets: Any = None) -> np.float32:
        from oracle import growth as og
        from plastax_amd.growth_config import GrowthConfig

        o = self.o
        loss = o.step(inputs, targets)
        while o.overflow:
            for level in range(len(o.static.level_capacities)):
                if self._free(level) == 0:
                    o.static, o.conns = og.grow_bucket(o.static, o.conns, level)
            cfg = GrowthConfig.of(o.plan.net, o.static)
            res = og.retry(cfg, o.units, o.conns, o.remainder, o.tail_start)
            o.conns = [{k: np.ascontiguousarray(v) for k, v in b.items()} for b in res.conns]
            o.grown += res.grown
            o.overflow = res.overflow
            o.needs_resort = o.needs_resort or res.needs_resort
            o.tail_start = res.tail_start
            o.remainder = res.remainder
            self._relayout()
        if not o.pipeline and o.needs_resort:
            o.static, o.units, o.conns, o.tail_start = og.resort(o.static, o.units, o.conns)
            o.units = {k: np.ascontiguousarray(v) for k, v in o.units.items()}
            o.conns = [{k: np.ascontiguousarray(v) for k, v in b.items()} for b in o.conns]
            o.needs_resort = False
            self._relayout()
        return loss
