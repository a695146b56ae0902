"""The structural phases on the device: PruneConn and add_conn growth.

Host orchestration of the kernels in csrc/structural.hip, mirroring the
reference's phases (phases.py:1444-1498 for PruneConn, :4490-5203 for
add_conn). Everything between the phase's inputs and its flags runs on the
GPU, stream-ordered, with device-side counts (no host round trip) until the
phase's four flags are read at its end:

1. candidates: the traced ``propose`` / ``score`` callback evaluated per
   site (``plx_site_eval``); shortlists rank units by importance with the
   radix sort;
2. validity (``plx_grow_filter``): window, direction, self-loops, source
   bucket, live endpoints, dedupe against the live edges (a sorted live-pair
   list and binary search); invalid candidates get score -inf;
3. dedupe within the step (``plx_grow_mark_repeats`` over a pair sort that
   is stable in score order);
4. the finite candidates, compacted in index order (``plx_compact``), sorted
   into the total order ``(-score, src, dst, index)``, level-major where the
   budget is per source level (``plx_sort``);
5. selection (``plx_grow_select``), init of the winners (site eval), claim
   and write (``plx_grow_claim``): TOPOLOGICAL winners take their bucket's
   free slots in order, PIPELINE winners their level's own dead slots and
   then the tail.

The arena is handled in its logical form: each bucket's columns in slot
order, concatenated into flat device columns (bucket ``b`` at
``[off_b, off_b + cap_b)``); the buckets handed back are views of them.
"""

from __future__ import annotations

import ctypes
import dataclasses
import pathlib
import warnings
from typing import Any

import numpy as np
import torch

from plastax_amd import _lib, _site
from plastax_amd._types import FROM_ID, TO_ID, Propagation
from plastax_amd.growth_config import GrowthConfig

Columns = dict[str, torch.Tensor]
_DIRECTION = {"any": 0, "deeper": 1, "same_or_deeper": 2}


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _bits_for(n: int) -> int:
    """Key bits that hold every value in [0, n]."""
    return max(1, int(n).bit_length())


def fill_prog(sp: _site.SiteProgram, units: Columns, conns: Columns | None, globals_: Any,
              physical_ids: bool = False) -> _lib.plx_site_prog:
    """The plx_site_prog of a traced site program over device columns
    (``physical_ids``: the conn id columns hold renumbered unit ids)."""
    p = _lib.plx_site_prog()
    p.ninstr = sp.ninstr
    p.nout = len(sp.out_kinds)
    code = sp.__dict__.get("_code_bytes")
    if code is None:  # (the code is fixed at trace time: packed once per program)
        code = np.ascontiguousarray(sp.flat_code(), dtype=np.int32).tobytes()
        sp.__dict__["_code_bytes"] = code
    ctypes.memmove(ctypes.addressof(p.code), code, len(code))
    for k, v in enumerate(sp.const_bits(globals_)):
        p.consts[k] = int(v)
    for f, name in enumerate(sp.unit_fields):
        col = units[name]
        assert col.is_contiguous()
        p.ufields[f] = col.data_ptr()
        p.ubytes[f] = 1 if col.element_size() == 1 else 4
    for f, name in enumerate(sp.conn_fields):
        assert conns is not None
        col = conns[name]
        p.cfields[f] = col.data_ptr()
        p.cbytes[f] = 1 if col.element_size() == 1 else 4
        if physical_ids and name in ("from_id", "to_id"):
            p.cbytes[f] |= _lib.PLX_SITE_ID_COLUMN
    return p


class Scratch:
    """Device scratch of the growth pipeline, allocated per call through
    torch's caching allocator."""

    def __init__(self, device: torch.device) -> None:
        self.device = device

    def i32(self, n: int) -> torch.Tensor:
        return torch.empty(max(int(n), 1), dtype=torch.int32, device=self.device)

    def f32(self, n: int) -> torch.Tensor:
        return torch.empty(max(int(n), 1), dtype=torch.float32, device=self.device)

    def u8(self, n: int) -> torch.Tensor:
        return torch.empty(max(int(n), 1), dtype=torch.uint8, device=self.device)

    def ints_for(self, n: int) -> torch.Tensor:
        return self.i32(int(_lib.load().plx_scratch_ints(int(n))))


# Site programs evaluated over at least this many sites run as their own
# compiled kernel (plx_site_compile; compiled once per program, device and
# launch shape); smaller launches interpret the program (plx_site_eval). Both
# give the same bits. "always" / "never" force either (tests).
COMPILE_SITES: str | int = 1 << 18
_CSRC = (pathlib.Path(__file__).resolve().parent / "csrc").as_posix().encode()


def _launch_shape(d: _lib.plx_site_desc) -> tuple:
    """What a compiled kernel fixes besides the code (plx_site_compile): the
    site kind, batched unit columns, which id arrays are set, the widths."""
    return (d.kind, d.batch > 1, bool(d.from_id), bool(d.to_id), bool(d.site_ids), bool(d.ids_logical),
            bool(d.ids_physical), tuple(d.prog.ubytes), tuple(d.prog.cbytes))


def compiled_site_handle(sp: _site.SiteProgram, d: _lib.plx_site_desc, device: torch.device) -> int | None:
    """The compiled kernel of a traced program for descriptor ``d``'s launch
    shape, kept on the program per (device, shape); None if hipRTC could not
    build it (the caller interprets the program instead, with a warning the
    first time)."""
    cache = sp.__dict__.setdefault("_compiled", {})
    dev = device.index if device.index is not None else torch.cuda.current_device()
    key = (dev, _launch_shape(d))
    if key in cache:
        return cache[key]
    lib = _lib.load()
    handle = ctypes.c_void_p()
    rc = lib.plx_site_compile(ctypes.byref(d), _CSRC, None, ctypes.byref(handle))
    if rc != 0:
        warnings.warn(f"site program not compiled, interpreted instead: {lib.plx_last_error().decode()[:500]}")
        cache[key] = None
        return None
    cache[key] = handle.value
    return handle.value


def compiled_forward_prune_handle(sp: _site.SiteProgram, prog: _lib.plx_site_prog, monoid: int,
                                  device: torch.device) -> int | None:
    """The fused forward + PruneConn kernel (plx_forward_prune_compile) of a
    traced predicate whose filled program is ``prog``, for ``monoid``, with
    the unit id arrays the fused forward passes; kept on the program per
    (device, monoid, field widths); None if hipRTC could not build it (the
    forward then interprets the predicate, with a warning the first time)."""
    cache = sp.__dict__.setdefault("_compiled_fwd", {})
    dev = device.index if device.index is not None else torch.cuda.current_device()
    key = (dev, int(monoid), tuple(prog.ubytes), tuple(prog.cbytes))
    if key in cache:
        return cache[key]
    d = _lib.plx_site_desc()
    d.prog = prog
    d.kind, d.batch, d.n, d.per = _lib_sites("EDGE"), 1, 1, 1
    d.ids_logical = d.ids_physical = ctypes.addressof(_ID_SHAPE)  # (only whether they are set)
    lib = _lib.load()
    handle = ctypes.c_void_p()
    rc = lib.plx_forward_prune_compile(ctypes.byref(d), int(monoid), _CSRC, None, ctypes.byref(handle))
    if rc != 0:
        warnings.warn(f"fused prune predicate not compiled, interpreted instead: "
                      f"{lib.plx_last_error().decode()[:500]}")
        cache[key] = None
        return None
    cache[key] = handle.value
    return handle.value


_ID_SHAPE = (ctypes.c_int32 * 1)()


class Kernels:
    """Thin wrappers of the structural entry points on one stream."""

    def __init__(self, device: torch.device, stream: int, timer: Any = None) -> None:
        self.lib = _lib.load()
        self.s = stream
        self.mem = Scratch(device)
        # Optional hook with begin(kind) / end(kind) around each entry-point
        # call (the benchmark records HIP events there).
        self.timer = timer

    def _begin(self, kind: str) -> None:
        if self.timer is not None:
            self.timer.begin(kind)

    def _end(self, kind: str) -> None:
        if self.timer is not None:
            self.timer.end(kind)

    def site_eval(self, sp: _site.SiteProgram, units: Columns, globals_: Any, *, n: int, kind: int,
                  per: int = 1, num_units: int, step: int = 0, net_seed: int = 0,
                  list_a: torch.Tensor | None = None, list_b: torch.Tensor | None = None,
                  from_id: torch.Tensor | None = None, to_id: torch.Tensor | None = None,
                  occ: torch.Tensor | None = None, n_dev: torch.Tensor | None = None,
                  outs: list[torch.Tensor] | None = None, conns: Columns | None = None,
                  or_into: torch.Tensor | None = None, kill_count: torch.Tensor | None = None,
                  site_ids: torch.Tensor | None = None, ids_logical: torch.Tensor | None = None,
                  ids_physical: torch.Tensor | None = None, batch: int = 1, sample: int = 0,
                  stamp: torch.Tensor | None = None, stamp_value: float = 0.0,
                  id_columns_logical: bool = False) -> None:
        """One site-program launch (plx_site_eval, or its compiled kernel).
        With ids_logical the unit columns and the id columns of `conns` are
        in the arena's numbering and translated to the caller's, unless
        `id_columns_logical`: the id columns passed already hold the
        caller's ids."""
        d = _lib.plx_site_desc()
        d.batch, d.sample = int(batch), int(sample)
        d.stamp, d.stamp_value = _ptr(stamp), float(stamp_value)
        d.prog = fill_prog(sp, units, conns, globals_,
                           physical_ids=ids_logical is not None and not id_columns_logical)
        d.n, d.kind, d.per, d.num_units = int(n), int(kind), int(per), int(num_units)
        d.step = int(np.array(int(step) & 0xFFFFFFFF, dtype=np.uint32).view(np.int32))
        d.net_seed = int(net_seed) & 0xFFFFFFFFFFFFFFFF
        d.list_a, d.list_b = _ptr(list_a), _ptr(list_b)
        d.from_id, d.to_id, d.occ, d.n_dev = _ptr(from_id), _ptr(to_id), _ptr(occ), _ptr(n_dev)
        for k, o in enumerate(outs or []):
            d.outs[k] = o.data_ptr()
        d.or_into = _ptr(or_into)
        d.kill_count, d.site_ids = _ptr(kill_count), _ptr(site_ids)
        d.ids_logical, d.ids_physical = _ptr(ids_logical), _ptr(ids_physical)
        policy = COMPILE_SITES
        compiled = policy == "always" or (policy != "never" and int(n) >= int(policy))
        handle = compiled_site_handle(sp, d, self.mem.device) if compiled else None
        self._begin("site_eval")
        if handle is not None:
            _lib.check(self.lib.plx_site_eval_compiled(handle, d, self.s), "plx_site_eval_compiled")
        else:
            _lib.check(self.lib.plx_site_eval(d, self.s), "plx_site_eval")
        self._end("site_eval")

    def compact(self, n: int, mode: int, flags: torch.Tensor, n_dev: torch.Tensor | None = None
                ) -> tuple[torch.Tensor, torch.Tensor]:
        out = self.mem.i32(n)
        count = self.mem.i32(1)
        scratch = self.mem.ints_for(n)
        _lib.check(self.lib.plx_compact(int(n), _ptr(n_dev), int(mode), flags.data_ptr(), out.data_ptr(),
                                        count.data_ptr(), scratch.data_ptr(), self.s), "plx_compact")
        return out, count

    def sort(self, vals: torch.Tensor, n_max: int, keys: list[tuple], n_dev: torch.Tensor | None = None,
             tag: str = "sort") -> None:
        """Stable sort of ``vals`` (in place) by ``keys`` (least significant
        first): (kind, bits, a, b[, bound]) per key."""
        if n_max == 0 or not keys:
            return
        d = _lib.plx_sort_desc()
        d.n_max, d.n_dev, d.nkeys = int(n_max), _ptr(n_dev), len(keys)
        for k, key in enumerate(keys):
            kind, bits, a, b = key[:4]
            d.keys[k].kind, d.keys[k].bits = int(kind), int(bits)
            d.keys[k].bound = int(key[4]) if len(key) > 4 else 0
            d.keys[k].a, d.keys[k].b = a.data_ptr(), _ptr(b)
        kb, ka, va = self.mem.i32(n_max), self.mem.i32(n_max), self.mem.i32(n_max)
        hist = self.mem.ints_for(n_max)
        d.vals, d.keys_buf, d.keys_alt, d.vals_alt, d.hist = (
            vals.data_ptr(), kb.data_ptr(), ka.data_ptr(), va.data_ptr(), hist.data_ptr())
        self._begin(tag)
        _lib.check(self.lib.plx_sort(d, self.s), "plx_sort")
        self._end(tag)

    def gather(self, idx: torch.Tensor, a: torch.Tensor, n_max: int, n_dev: torch.Tensor | None) -> torch.Tensor:
        out = self.mem.i32(n_max)
        _lib.check(self.lib.plx_gather_i32(int(n_max), _ptr(n_dev), idx.data_ptr(), a.data_ptr(), out.data_ptr(),
                                           self.s), "plx_gather_i32")
        return out

    def iota(self, n: int) -> torch.Tensor:
        return torch.arange(max(int(n), 1), dtype=torch.int32, device=self.mem.device)


@dataclasses.dataclass
class Remainder:
    """A growth phase's winners on the device, kept for its same-step retry
    (the reference's GrowthRemainder, phases.py:2776-2816): the winner list
    (level-major, count in ``nwin``), the candidate columns it indexes, the
    init values of every winner, and which growable winners found no slot."""

    nc: int
    winners: torch.Tensor
    nwin: torch.Tensor
    src: torch.Tensor
    dst: torch.Tensor
    score: torch.Tensor
    init_outs: list[torch.Tensor]
    dropped: torch.Tensor
    nseg: int


_OFFS_CACHE: dict[tuple, torch.Tensor] = {}


class ClaimedSlots:
    """The flat slots a claim filled, appended in no particular order
    (``plx_grow_claim``'s claimed_out): ``count`` (device int32) of them in
    ``slots``, at most ``bound``; ``offs`` are the buckets' flat starts.
    ``split`` sorts them into each bucket's ascending relative slots."""

    def __init__(self, slots: torch.Tensor, count: torch.Tensor, bound: int, offs: list[int]) -> None:
        self.slots, self.count, self.bound, self.offs = slots, count, int(bound), list(offs)

    def split(self, lib: Any, stream: int) -> tuple[torch.Tensor, torch.Tensor]:
        """(out [nb, max(bound, 1)], counts [nb]): bucket b's claimed slots
        less its start, ascending, in out[b, :counts[b]]."""
        dev = self.slots.device
        nb = len(self.offs) - 1
        region = max(self.bound, 1)
        out = torch.empty((nb, region), dtype=torch.int32, device=dev)
        counts = torch.empty(nb, dtype=torch.int32, device=dev)
        key = (tuple(self.offs), dev)
        offs = _OFFS_CACHE.get(key)
        if offs is None:  # (one host-to-device copy per arena shape, not per step)
            offs = _OFFS_CACHE[key] = torch.tensor(self.offs, dtype=torch.int64, device=dev)
        _lib.check(lib.plx_claimed_split(self.bound, self.count.data_ptr(), self.slots.data_ptr(), nb,
                                         offs.data_ptr(), region, out.data_ptr(), counts.data_ptr(), stream),
                   "plx_claimed_split")
        return out, counts


class GrowthOutcome:
    """A growth phase's result: the new buckets, whether it ran, and its
    flags. A claim leaves the flags on the device (``flags``: int32 grown,
    overflow, needs_resort, tail slots used and, for PIPELINE, the new tail
    start), read on first access of ``grown`` / ``overflow`` /
    ``needs_resort`` / ``tail_start``; a step passes them on unread."""

    def __init__(self, conns: tuple[Columns, ...], grown: int = 0, overflow: bool = False,
                 needs_resort: bool = False, tail_start: Any = 0, fired: bool = False, *,
                 flags: torch.Tensor | None = None) -> None:
        self.conns = conns
        self.fired = fired
        self.flags = flags
        self._tail_in = tail_start  # host int or a device int32[1] (PIPELINE)
        self._host = None if flags is not None else (int(grown), bool(overflow), bool(needs_resort), tail_start)

    def _values(self) -> tuple[int, bool, bool, int]:
        if self._host is None:
            got = self.flags.cpu().tolist()
            tail = got[4] if len(got) > 4 else self._tail_in
            self._host = (int(got[0]), bool(got[1]), bool(got[2]), int(tail))
        return self._host

    grown = property(lambda self: self._values()[0])
    overflow = property(lambda self: self._values()[1])
    needs_resort = property(lambda self: self._values()[2])
    tail_start = property(lambda self: int(self._values()[3]))


def flatten(conns: tuple[Columns, ...]) -> tuple[Columns, list[int]]:
    """One flat column per field, the buckets end to end; offsets."""
    caps = [int(next(iter(b.values())).shape[0]) for b in conns]
    offs = [0]
    for c in caps:
        offs.append(offs[-1] + c)
    if len(conns) == 1:
        flat = {name: col.contiguous() for name, col in conns[0].items()}
    else:
        flat = {name: torch.cat([b[name] for b in conns]).contiguous() for name in conns[0]}
    return flat, offs


def unflatten(flat: Columns, offs: list[int]) -> tuple[Columns, ...]:
    return tuple({name: col[offs[b] : offs[b + 1]] for name, col in flat.items()} for b in range(len(offs) - 1))


class PruneConnPhase:
    """``dead |= predicate(u, c, cid, g)`` over every slot of every bucket
    (phases.py:1444-1498), one site-program launch per bucket."""

    def __init__(self, net: Any, static: Any, globals_: Any) -> None:
        self.static = static
        unit_dtypes = {s.name: np.dtype(s.dtype) for s in static.unit_fields}
        conn_dtypes = {s.name: np.dtype(s.dtype) for s in static.conn_fields}
        self.prog = _site.trace_predicate(net.prune_conn, unit_dtypes, conn_dtypes, globals_)

    def run(self, k: Kernels, units: Columns, conns: tuple[Columns, ...], globals_: Any,
            kill_count: torch.Tensor | None = None) -> None:
        """On the logical arena (caller's unit ids, slot order)."""
        n_units = int(next(iter(units.values())).shape[0])
        for bucket in conns:
            cap = int(bucket["dead"].shape[0])
            if cap == 0:
                continue
            k.site_eval(self.prog, units, globals_, n=cap, kind=_lib_sites("EDGE"), num_units=n_units,
                        conns=bucket, or_into=bucket["dead"], kill_count=kill_count)

    def run_physical(self, k: Kernels, arena: Any, units: Columns, globals_: Any,
                     kill_count: torch.Tensor | None = None) -> None:
        """On the step's physical arena: positions of bucket b are
        [base_b, base_b + cap_b), unit columns and the id columns are in the
        arena's unit order; the program still sees the caller's ids and each
        edge's logical slot (arena.slot). An edge killed in a bucket whose
        Adam step count is kept as one number gets that number in its own
        column (arena.stamp_target), so no host read follows the pass."""
        n_units = int(next(iter(units.values())).shape[0])
        # A program that reads FROM_ID / TO_ID reads them in the caller's
        # numbering: a churn arena keeps the caller's ids (no translation at
        # all), a tiled one keeps translated copies (Arena.logical_ids) so
        # that no edge pays two id gathers.
        churn = bool(getattr(arena, "churn", False))
        reads_ids = bool({FROM_ID.name, TO_ID.name} & set(self.prog.conn_fields))
        logical = arena.logical_ids() if reads_ids and not churn else None
        for b in range(arena.num_buckets):
            base, cap = arena.bases[b], arena.caps[b]
            if cap == 0:
                continue
            view = {name: col[base : base + cap] for name, col in arena.cols.items()}
            if logical is not None:
                view.update({name: col[base : base + cap] for name, col in logical.items()})
            stamp, value = arena.stamp_target(b)
            k.site_eval(self.prog, units, globals_, n=cap, kind=_lib_sites("EDGE"), num_units=n_units,
                        conns=view, or_into=view["dead"], kill_count=kill_count,
                        # (the logical slot only where the program reads cid's value)
                        site_ids=arena.slot[base : base + cap] if self.prog.uses_role("cid") else None,
                        ids_logical=None if churn else arena.uperm32,
                        ids_physical=None if churn else arena.uinv32, stamp=stamp, stamp_value=value,
                        id_columns_logical=logical is not None)


class ConnUpdatePhase:
    """A user UpdateConn (phases.py:1196-1242, sweep.py:488-532): every
    bucket's incoming pass, then every bucket's outgoing pass, each an edge
    program whose writes land on the edge's own row (dead rows keep theirs)."""

    def __init__(self, net: Any, static: Any, globals_: Any) -> None:
        unit_dtypes = {s.name: np.dtype(s.dtype) for s in static.unit_fields}
        uc = net.update_conn
        self.passes = [_site.trace_conn_update(getattr(uc, d), d, unit_dtypes, static.conn_fields, globals_)
                       for d in ("incoming", "outgoing")]

    def run_physical(self, k: Kernels, arena: Any, units: Columns, globals_: Any) -> None:
        """On the step's physical arena, over each bucket's positions that
        held live edges when it was laid out ([base, base + live); a slot
        dead then is not laid out with its values and keeps them, and one
        tombstoned since reads its DEAD and keeps its row). The programs see
        the caller's ids and each edge's logical slot."""
        n_units = int(next(iter(units.values())).shape[0])
        for prog, names in self.passes:
            if not names:
                continue
            for b in range(arena.num_buckets):
                base, live = arena.bases[b], arena.lives[b]
                if live == 0:
                    continue
                view = {name: col[base : base + live] for name, col in arena.cols.items()}
                k.site_eval(prog, units, globals_, n=live, kind=_lib_sites("EDGE"), num_units=n_units,
                            conns=view, outs=[view[name] for name in names],
                            from_id=view["from_id"], to_id=view["to_id"],
                            site_ids=arena.slot[base : base + live], ids_logical=arena.uperm32,
                            ids_physical=arena.uinv32)


def _lib_sites(name: str) -> int:
    return {"UNIT": 0, "GLOBAL": 1, "CONN": 2, "GRID": 3, "PAIRS": 4, "EDGE": 5}[name]


class AddConnPhase:
    """One add_conn phase on the device (phases.py:4490-5203)."""

    def __init__(self, net: Any, static: Any, globals_: Any) -> None:
        self.net = net
        self.ac = net.add_conn
        self.static = static
        self.cfg = GrowthConfig.of(net, static)
        self.interval = int(getattr(net, "structural_interval", 1))
        unit_dtypes = {s.name: np.dtype(s.dtype) for s in static.unit_fields}
        conn_dtypes = {s.name: np.dtype(s.dtype) for s in static.conn_fields}
        cfg = self.cfg
        if cfg.propose:
            self.cand_prog = _site.trace_propose(self.ac, cfg.proposer, unit_dtypes, conn_dtypes, globals_)
        else:
            self.cand_prog = _site.trace_score(self.ac, unit_dtypes, globals_)
        self.imp_prog = _site.trace_importance(self.ac, unit_dtypes, globals_) if cfg.shortlist else None
        self.init_prog, self.init_names = _site.trace_init(self.ac, unit_dtypes, static.conn_fields, globals_)
        self.remainder: Remainder | None = None
        # (flags of the last PIPELINE claim, a host bound on the tail start
        # it wrote into flags[4])
        self._tail_hint: tuple[torch.Tensor, int] | None = None
        # a bound on the slots the last claim filled (sizes the next relayout)
        self.claim_bound: int | None = None
        # set by the caller: the claim also lists the slots it fills
        # (ClaimedSlots, for a merged relayout; None when the bound is too
        # large for plx_claimed_split or the list was not asked for)
        self.want_claimed = False
        self.claimed: ClaimedSlots | None = None
        # (a level column, a bound on its deepest level): read once, then
        # carried through the add_unit phases that derive new columns
        self._level_hint: tuple[torch.Tensor, int] | None = None

    def claims_listable(self, level: torch.Tensor) -> bool:
        """Whether the claim's filled slots can be listed for a merged
        relayout: the bound on them the claim will use (its winners' budget,
        ``claim_bound``), known now without a host read, fits
        plx_claimed_split. ``level``: the level column the phase will run
        with (PIPELINE: its carried bound gives the segments)."""
        cfg = self.cfg
        if cfg.step_scope:
            bound = int(cfg.k)
        elif cfg.pipeline:
            hint = self._level_hint
            if hint is None or hint[0] is not level:
                return False
            bound = (int(hint[1]) + 1) * int(cfg.k)
        else:
            bound = int(cfg.num_buckets) * int(cfg.k)
        if cfg.max_new_per_step:
            bound = min(bound, int(cfg.max_new_per_step))
        return max(0, bound) <= _lib.PLX_CLAIMED_SPLIT_MAX

    def level_bound(self, level: torch.Tensor) -> int:
        """A bound on the deepest level of ``level``: the carried one when
        this is the column it was carried to, else one host read."""
        hint = self._level_hint
        if hint is not None and hint[0] is level:
            return hint[1]
        bound = int(level.max().item()) if level.numel() else 0
        self._level_hint = (level, bound)
        return bound

    def carry_level_bound(self, old: torch.Tensor, new: torch.Tensor, bound_after: Any) -> None:
        """add_unit derived the column ``new`` from ``old``:
        ``bound_after(b)`` bounds its deepest level given ``old``'s bound b
        (nothing carried when ``old``'s bound is not known)."""
        hint = self._level_hint
        if hint is not None and hint[0] is old:
            self._level_hint = (new, int(bound_after(hint[1])))

    # -- helpers ---------------------------------------------------------------
    def _top_units(self, k: Kernels, masked: torch.Tensor, m: int, n: int) -> torch.Tensor:
        """lax.top_k's ids: descending value, ties to the lower id."""
        order = k.iota(n)
        k.sort(order, n, [(1, 32, masked, None)])  # PLX_KEY_SCORE
        return order[:m]

    def _importance(self, k: Kernels, units: Columns, globals_: Any, n: int) -> torch.Tensor:
        imp = k.mem.f32(n)
        k.site_eval(self.imp_prog, units, globals_, n=n, kind=_lib_sites("UNIT"), per=1, num_units=n, outs=[imp])
        return imp

    def _mask(self, k: Kernels, imp: torch.Tensor, units: Columns, mode: int, b: int) -> torch.Tensor:
        n = int(imp.shape[0])
        out = k.mem.f32(n)
        pruned = units.get("pruned")
        gap = self.cfg.max_level_gap if mode == 1 else 0
        direction = _DIRECTION[self.cfg.direction] if mode == 1 else 0
        _lib.check(k.lib.plx_mask_importance(n, imp.data_ptr(), units["level"].data_ptr(), _ptr(pruned), mode, b,
                                             gap, direction, out.data_ptr(), k.s), "plx_mask_importance")
        return out

    # -- the phase --------------------------------------------------------------
    def run(self, k: Kernels, units: Columns, conns: tuple[Columns, ...], *, step: int, globals_: Any,
            tail_start: Any = 0, units_added: int = 0, needs_resort: Any = False) -> GrowthOutcome:
        """One growth phase. ``tail_start``: an int, or (PIPELINE) a device
        int32[1] such as the last outcome's ``flags[4:5]``. ``needs_resort``:
        the flag before the phase (a bool, or a pending (device tensor,
        index)); the outcome's needs_resort is it OR the claim's."""
        cfg = self.cfg
        if not cfg.fires(self.ac, step=step, interval=self.interval, units_added=units_added, globals_=globals_):
            return GrowthOutcome(conns, 0, False, False, tail_start, False)
        n = cfg.num_units
        nb = cfg.num_buckets
        flat, offs = flatten(conns)
        total_slots = offs[-1]
        level = units["level"]
        pruned = units.get("pruned")
        seed, dev = int(self.static.seed), level.device
        INT_MAX = 0x7FFFFFFF
        # PIPELINE: the levels bound the per-level segments (they run up to
        # the unit count). A bound on the deepest level sizes them: read once,
        # then carried (level_bound); a bound above the deepest level only
        # adds empty segments.
        max_level = self.level_bound(level) if cfg.pipeline else 0

        # 1. candidates
        grid_sq = 0
        proposer_idx = proposer_dead = None
        per = 1
        if cfg.propose:
            P = cfg.proposals
            per = P
            if cfg.proposer == "per_unit":
                nc, kind = n * P, _lib_sites("UNIT")
                extra = {}
                proposer_dead = pruned
            elif cfg.proposer == "global":
                nc, kind, extra = P, _lib_sites("GLOBAL"), {}
            else:
                nc, kind = total_slots * P, _lib_sites("CONN")
                perm = k.iota(total_slots)
                bits = _bits_for(n)
                k.sort(perm, total_slots, [(4, bits, flat["to_id"], flat["dead"]),
                                           (4, bits, flat["from_id"], flat["dead"])])
                occ = k.mem.i32(total_slots)
                _lib.check(k.lib.plx_occurrence(total_slots, perm.data_ptr(), flat["from_id"].data_ptr(),
                                                flat["to_id"].data_ptr(), occ.data_ptr(), k.s), "plx_occurrence")
                extra = dict(list_a=perm, from_id=flat["from_id"], to_id=flat["to_id"], occ=occ, conns=flat)
                proposer_idx, proposer_dead = perm, flat["dead"]
            src, dst, score = k.mem.i32(nc), k.mem.i32(nc), k.mem.f32(nc)
            k.site_eval(self.cand_prog, units, globals_, n=nc, kind=kind, per=P, num_units=n, step=step,
                        net_seed=seed, outs=[src, dst, score], **extra)
        else:
            if cfg.per_level:
                M = cfg.pool_side
                imp = self._importance(k, units, globals_, n)
                src_lists = torch.cat([self._top_units(k, self._mask(k, imp, units, 0, b), M, n) for b in range(nb)])
                dst_lists = torch.cat([self._top_units(k, self._mask(k, imp, units, 1, b), M, n) for b in range(nb)])
                side, ngrids = M, nb
                grid_sq = M * M
            elif cfg.shortlist:
                M = cfg.pool_side
                imp = self._importance(k, units, globals_, n)
                top = self._top_units(k, self._mask(k, imp, units, 2, 0), M, n)
                src_lists = dst_lists = top
                side, ngrids = M, 1
            else:
                src_lists = dst_lists = k.iota(n)
                side, ngrids = n, 1
            nc = ngrids * side * side
            if nc > INT_MAX:
                raise ValueError(f"add_conn: {nc} candidates exceed 2^31 - 1; use a shortlist")
            src, dst, score = k.mem.i32(nc), k.mem.i32(nc), k.mem.f32(nc)
            pairs = [src, dst]
            k.site_eval(_pairs_prog(), units, globals_, n=nc, kind=_lib_sites("GRID"), per=side, num_units=n,
                        list_a=src_lists, list_b=dst_lists, outs=pairs)
            k.site_eval(self.cand_prog, units, globals_, n=nc, kind=_lib_sites("GRID"), per=side, num_units=n,
                        list_a=src_lists, list_b=dst_lists, outs=[score])

        # 2. validity
        f = _lib.plx_grow_filter_desc()
        f.n, f.grid_sq, f.num_units, f.num_buckets = nc, grid_sq, n, nb
        f.pipeline = int(cfg.pipeline)
        f.max_level_gap = min(cfg.max_level_gap, INT_MAX)
        f.direction = _DIRECTION[cfg.direction]
        f.allow_self_loops = int(cfg.allow_self_loops)
        f.check_range = int(cfg.propose)
        f.per = per
        f.src, f.dst, f.score, f.level, f.pruned = src.data_ptr(), dst.data_ptr(), score.data_ptr(), \
            level.data_ptr(), _ptr(pruned)
        f.proposer_idx, f.proposer_dead = _ptr(proposer_idx), _ptr(proposer_dead)
        if cfg.dedupe_live and total_slots:
            live_idx, nlive = k.compact(total_slots, 1, flat["dead"])  # PLX_FLAG_U8_ZERO
            if cfg.pipeline:
                bucket_id = torch.zeros(total_slots, dtype=torch.int32, device=dev)
            else:
                caps = torch.tensor([offs[b + 1] - offs[b] for b in range(nb)], device=dev)
                bucket_id = torch.repeat_interleave(torch.arange(nb, dtype=torch.int32, device=dev), caps)
            bits = _bits_for(n)
            k.sort(live_idx, total_slots, [(0, bits, flat["to_id"], None), (0, bits, flat["from_id"], None),
                                           (0, _bits_for(nb), bucket_id, None)], n_dev=nlive)
            f.nlive, f.nlive_dev, f.live_idx = total_slots, nlive.data_ptr(), live_idx.data_ptr()
            f.live_bucket, f.live_src, f.live_dst = bucket_id.data_ptr(), flat["from_id"].data_ptr(), \
                flat["to_id"].data_ptr()
        _lib.check(k.lib.plx_grow_filter(f, k.s), "plx_grow_filter")

        pair_keys = self._pair_keys(src, dst, n)
        # 3. dedupe within the step
        if cfg.dedupe_step:
            fin, nfin = k.compact(nc, 2, score)  # PLX_FLAG_FINITE
            k.sort(fin, nc, [(1, 32, score, None), *pair_keys], n_dev=nfin)
            _lib.check(k.lib.plx_grow_mark_repeats(nc, nfin.data_ptr(), fin.data_ptr(), src.data_ptr(),
                                                   dst.data_ptr(), score.data_ptr(), k.s), "plx_grow_mark_repeats")

        # 4. total order of the finite candidates
        order, nord = k.compact(nc, 2, score)
        per_segment = not cfg.step_scope
        nseg = max_level + 1 if cfg.pipeline else nb
        level_key = (2, _bits_for(nseg - 1), src, level, n)  # PLX_KEY_LEVEL_OF, ids clamped to [0, n)
        keys = [*pair_keys, (1, 32, score, None)]
        if per_segment:
            keys.append(level_key)
        k.sort(order, nc, keys, n_dev=nord, tag="total_order")
        # (for measurement: the sorted count and the 8-bit digit passes)
        self.last_sort = (nord, sum((int(key[1]) + 7) // 8 for key in keys))

        # 5. selection
        win = k.mem.u8(nc)
        first = k.mem.i32(nseg)
        _lib.check(k.lib.plx_grow_select(nc, nord.data_ptr(), order.data_ptr(), src.data_ptr(), level.data_ptr(),
                                         int(per_segment), int(cfg.k), nseg, first.data_ptr(), win.data_ptr(), k.s),
                   "plx_grow_select")
        wpos, nwin = k.compact(nc, 0, win, n_dev=nord)  # PLX_FLAG_U8
        winners = k.gather(wpos, order, nc, nwin)
        if not per_segment:
            k.sort(winners, nc, [level_key], n_dev=nwin)

        # init of the winners
        wsrc = k.gather(winners, src, nc, nwin)
        wdst = k.gather(winners, dst, nc, nwin)
        init_outs = [k.mem.i32(nc) for _ in self.init_names]
        if self.init_names:
            k.site_eval(self.init_prog, units, globals_, n=nc, kind=_lib_sites("PAIRS"), num_units=n,
                        list_a=wsrc, list_b=wdst, n_dev=nwin, outs=init_outs)

        # 6. claim and write
        threshold = None
        if cfg.selection == "threshold":
            threshold = float(np.float32(np.asarray(self.ac.threshold(globals_))))
        rem = Remainder(nc, winners, nwin, src, dst, score, init_outs, k.mem.i32(nc), nseg)
        self.remainder = rem
        return self._claim(k, level, conns, flat, offs, tail_start, rem, threshold=threshold,
                           needs_resort=needs_resort)

    def retry(self, k: Kernels, units: Columns, conns: tuple[Columns, ...], *, tail_start: Any) -> GrowthOutcome:
        """Claim the winners the last phase dropped into ``conns`` (its buckets
        regrown by the caller), with the values that phase computed, in the
        total order (build_growth_retry, phases.py:5206-5281). No other
        stage re-runs; ``grown`` counts only this claim's commits."""
        rem = self.remainder
        if rem is None:
            raise RuntimeError("retry: the last add_conn phase left no remainder")
        flat, offs = flatten(conns)
        growable = rem.dropped.clone()
        return self._claim(k, units["level"], conns, flat, offs, tail_start, rem, growable_in=growable)

    def _claim(self, k: Kernels, level: torch.Tensor, conns: tuple[Columns, ...], flat: Columns, offs: list[int],
               tail_start: Any, rem: "Remainder", *, threshold: float | None = None,
               growable_in: torch.Tensor | None = None, needs_resort: Any = False) -> GrowthOutcome:
        cfg = self.cfg
        n, nb, nc, nseg = cfg.num_units, cfg.num_buckets, rem.nc, rem.nseg
        total_slots = offs[-1]
        dev = level.device
        c = _lib.plx_grow_claim_desc()
        c.n_max, c.n_dev, c.winners = nc, rem.nwin.data_ptr(), rem.winners.data_ptr()
        c.src, c.dst, c.score, c.level = rem.src.data_ptr(), rem.dst.data_ptr(), rem.score.data_ptr(), level.data_ptr()
        c.pipeline, c.num_buckets, c.num_levels = int(cfg.pipeline), nb, nseg
        if threshold is not None:
            c.has_threshold = 1
            c.threshold = threshold
        c.max_new_per_step = int(cfg.max_new_per_step or 0)
        c.capacity = total_slots
        keep: list[torch.Tensor] = []
        tail_dev = None
        if cfg.pipeline:
            # Each level's own dead slots (below the tail, by the level of
            # their former source), in slot order, level after level. The
            # tail start is a device int32 (the last claim's result, or the
            # caller's value), so the lists are sized by the arena's slots
            # and counted on the device.
            # The lists are sized by a host bound on the tail: exact for a host
            # value; for the last claim's device tail, that claim's bound
            # plus its winner budget (tail slots used <= winners); else the
            # arena's slots.
            if isinstance(tail_start, torch.Tensor):
                tail_dev = tail_start
                hint = self._tail_hint
                span = total_slots
                if hint is not None and tail_dev.data_ptr() == hint[0].data_ptr() + 16:
                    span = hint[1]
            else:
                span = int(tail_start)
                tail_dev = torch.tensor([span], dtype=torch.int32, device=dev)
            span = max(0, min(total_slots, span))
            c.tail_dev = tail_dev.data_ptr()
            own, nown = k.compact(span, 0, flat["dead"], n_dev=tail_dev)  # PLX_FLAG_U8 over [0, tail)
            k.sort(own, span, [(2, _bits_for(nseg - 1), flat["from_id"], level, n)], n_dev=nown)
            domain = k.mem.i32(span)
            _lib.check(k.lib.plx_gather_level(span, nown.data_ptr(), own.data_ptr(), flat["from_id"].data_ptr(),
                                              level.data_ptr(), n, domain.data_ptr(), k.s), "plx_gather_level")
            count, start = k.mem.i32(nseg), k.mem.i32(nseg)
            lscratch = k.mem.ints_for(nseg)
            _lib.check(k.lib.plx_level_counts(span, nown.data_ptr(), domain.data_ptr(), nseg,
                                              count.data_ptr(), start.data_ptr(), lscratch.data_ptr(), k.s),
                       "plx_level_counts")
            c.own_slots, c.own_start, c.own_count = own.data_ptr(), start.data_ptr(), count.data_ptr()
            keep += [domain, own, nown, count, start, lscratch, tail_dev]
        else:
            c.tail_start = int(tail_start)
            free, nfree = k.compact(total_slots, 0, flat["dead"])
            off = torch.tensor(offs, dtype=torch.int64, device=dev)
            info = k.mem.i32(2 * nb)
            _lib.check(k.lib.plx_bucket_free(nb, off.data_ptr(), free.data_ptr(), nfree.data_ptr(), info.data_ptr(),
                                             k.s), "plx_bucket_free")
            c.free_slots, c.free_info = free.data_ptr(), info.data_ptr()
            keep += [free, nfree, off, info]
        c.from_id, c.to_id, c.dead = flat["from_id"].data_ptr(), flat["to_id"].data_ptr(), flat["dead"].data_ptr()
        ncols = 0
        for spec in self.static.conn_fields:
            if spec.name in ("from_id", "to_id", "dead"):
                continue
            col = flat[spec.name]
            gc = c.cols[ncols]
            gc.ptr = col.data_ptr()
            gc.bytes = 1 if col.element_size() == 1 else 4
            if spec.name in self.init_names:
                gc.init_slot = self.init_names.index(spec.name)
            else:
                gc.init_slot = -1
                gc.default_bits = _default_bits(spec)
            ncols += 1
        c.ncols = ncols
        for j, o in enumerate(rem.init_outs):
            c.init_out[j] = o.data_ptr()
        # grown, overflow, needs_resort, tail slots used (+ the new tail start)
        flags = torch.zeros(5 if tail_dev is not None else 4, dtype=torch.int32, device=dev)
        if isinstance(needs_resort, tuple):  # the claim ORs into the flag it starts from
            t, i = needs_resort
            flags[2:3].copy_(t[i : i + 1])
        elif needs_resort:
            flags[2:3].fill_(1)
        scratch = k.mem.i32(8 * nc + int(k.lib.plx_scratch_ints(nc)))
        c.flags, c.scratch = flags.data_ptr(), scratch.data_ptr()
        c.growable_in, c.dropped_out = _ptr(growable_in), rem.dropped.data_ptr()
        # claims are winners: a bound on the slots this claim can fill
        winners_max = max(0, nseg * int(cfg.k) if not cfg.step_scope else int(cfg.k))
        if cfg.max_new_per_step:
            winners_max = min(winners_max, int(cfg.max_new_per_step))
        self.claim_bound = min(winners_max, nc)
        self.claimed = None
        if self.want_claimed and self.claim_bound <= _lib.PLX_CLAIMED_SPLIT_MAX:
            # the filled slots, appended by the claim (for a merged relayout)
            lst = k.mem.i32(max(self.claim_bound, 1))
            cnt = torch.zeros(1, dtype=torch.int32, device=dev)
            c.claimed_out, c.claimed_n, c.claimed_cap = lst.data_ptr(), cnt.data_ptr(), self.claim_bound
            self.claimed = ClaimedSlots(lst, cnt, self.claim_bound, offs)
        _lib.check(k.lib.plx_grow_claim(c, k.s), "plx_grow_claim")
        if tail_dev is not None:
            # the new tail (flags[4]) is at most the old bound plus the winners
            self._tail_hint = (flags, span + self.claim_bound)
        out = GrowthOutcome(unflatten(flat, offs), tail_start=tail_start, fired=True, flags=flags)
        if cfg.on_overflow == "error" and out.overflow:  # (this policy reads the flags here)
            raise RuntimeError("add_conn overflow: selected candidates exceeded the free connection capacity")
        return out

    @staticmethod
    def _pair_keys(src: torch.Tensor, dst: torch.Tensor, n: int) -> list[tuple[int, int, torch.Tensor, Any]]:
        """Sort keys ordering by (src, dst), least significant first."""
        if n <= 1 << 16:
            return [(3, 32, src, dst)]  # PLX_KEY_PAIR16
        bits = _bits_for(n)
        return [(0, bits, dst, None), (0, bits, src, None)]


def _default_bits(spec: Any) -> int:
    v = np.asarray(spec.default).astype(spec.dtype)
    if v.dtype == np.bool_:
        return int(bool(v))
    if v.dtype.itemsize != 4:
        raise TypeError(f"conn column {spec.name!r}: only 32-bit and bool columns can grow")
    return int(v.view(np.uint32))


_PAIRS: _site.SiteProgram | None = None


def _pairs_prog() -> _site.SiteProgram:
    """The site program writing a grid site's (src, dst)."""
    global _PAIRS
    if _PAIRS is None:
        _PAIRS = _site.compile_site_program([(_site.idx("src"), "i"), (_site.idx("dst"), "i")], roles=("src", "dst"))
    return _PAIRS
