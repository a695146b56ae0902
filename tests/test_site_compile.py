"""Compiled site programs (plx_site_compile): the generated kernel source
compiles with hipRTC for gfx950 under the library's floating-point flags,
for a program holding every opcode of the site machine and for traced
policies (a PruneConn hash predicate, a Box-Muller proposer, the SET
proposer's table reads), under each launch shape the kernel fixes (site
kind, batched unit columns, id arrays, byte-wide fields). Compile only -- no device is needed; the device
runs of compiled programs against the oracle are in
test_gpu_site_compiled.py."""

from __future__ import annotations

import ctypes
import pathlib

import numpy as np
import pytest

import plastax_amd as px
import plastax_amd.numpy as jnp
from plastax_amd import _lib, _site

CSRC = (pathlib.Path(_lib.__file__).resolve().parent / "csrc").as_posix().encode()


def _prog(code: list[tuple[int, int, int, int]], nout: int) -> _lib.plx_site_prog:
    p = _lib.plx_site_prog()
    p.ninstr = len(code)
    p.nout = nout
    for k, ins in enumerate(code):
        for j in range(4):
            p.code[4 * k + j] = int(ins[j])
    return p


_DUMMY = (ctypes.c_int32 * 1)()


def _desc(p: _lib.plx_site_prog, kind: int = 5, batch: int = 1, ids: bool = False,
          ends: bool = False) -> _lib.plx_site_desc:
    """A descriptor of program p for compiling only: the pointers that fix
    the shape are set to a dummy host address (nothing is launched)."""
    d = _lib.plx_site_desc()
    d.prog = p
    d.kind, d.batch, d.n, d.per = kind, batch, 1, 1
    addr = ctypes.addressof(_DUMMY)
    if ids:
        d.ids_logical = d.ids_physical = d.site_ids = addr
    if ends:
        d.from_id = d.to_id = addr
    return d


def _compile(p: _lib.plx_site_prog, **shape) -> None:
    lib = _lib.load()
    rc = lib.plx_site_compile(ctypes.byref(_desc(p, **shape)), CSRC, b"gfx950", None)
    assert rc == 0, lib.plx_last_error().decode()[:3000]


def _traced(sp: _site.SiteProgram) -> _lib.plx_site_prog:
    code = sp.flat_code().reshape(-1, 4)
    return _prog([tuple(int(v) for v in row) for row in code], len(sp.out_kinds))


def test_every_opcode_compiles() -> None:
    ops = sorted(set(_site.SOP.values()) - {_site.SOP["out"]})
    code = [(op, k % 32, 1 + k % 4, 2 + k % 8) for k, op in enumerate(ops)]
    code += [(_site.SOP["out"], 0, 3, 0), (_site.SOP["out"], 1, 5, 0)]
    assert len(code) <= _site.MAX_SINSTR
    p = _prog(code, 2)
    _compile(p)
    for f in range(3):  # byte-wide (bool) columns and id columns
        p.ubytes[f], p.cbytes[f] = 1, 4 | _lib.PLX_SITE_ID_COLUMN
    for shape in (dict(kind=0, batch=8, ids=True), dict(kind=5, ids=True, ends=True), dict(kind=2),
                  dict(kind=3), dict(kind=4), dict(kind=1)):
        _compile(p, **shape)


def test_traced_policies_compile() -> None:
    class HashPrune(px.PruneConn):
        def predicate(self, u, c, cid, g):
            h = c[px.FROM_ID, cid] * jnp.int32(7) + c[px.TO_ID, cid] * jnp.int32(13) + g["step"]
            return (h % jnp.int32(1048573)) == jnp.int32(0)

    class NormalRule(px.ProposeAddConn):
        proposer = "per_unit"
        proposals_per_proposer = 4

        def propose(self, u, i, j, g, rng):
            z = rng.normal()
            dst = (jnp.abs(z) * jnp.float32(700.0)).astype(jnp.int32) % 3000
            return px.Proposal(i, dst, rng.normal() + jnp.cos(u[px.ACTIVATION, i]))

    class Tables(px.ProposeAddConn):
        proposer = "per_unit"
        proposals_per_proposer = 4

        def __init__(self):
            self.start = jnp.asarray(np.int32([4, 10, 16]))
            self.width = jnp.asarray(np.int32([6, 6, 0]))

        def propose(self, u, i, j, g, rng):
            layer = jnp.sum(i >= self.start)
            w = self.width[layer]
            dst = self.start[layer] + jnp.minimum((rng.uniform() * w.astype(jnp.float32)).astype(jnp.int32), w - 1)
            return px.Proposal(i, dst, jnp.where(w > 0, rng.uniform(), -jnp.inf))

    udt = {"activation": np.dtype(np.float32), "level": np.dtype(np.int32)}
    cdt = {"from_id": np.dtype(np.int32), "to_id": np.dtype(np.int32), "weight": np.dtype(np.float32)}
    progs = [
        _site.trace_predicate(HashPrune(), udt, cdt, {"step": np.int32(0)}),
        _site.trace_propose(NormalRule(), "per_unit", udt, cdt, None),
        _site.trace_propose(Tables(), "per_unit", udt, cdt, None),
    ]
    _compile(_traced(progs[0]), kind=5, ends=True)
    for sp in progs[1:]:
        _compile(_traced(sp), kind=0)


def test_compile_rejects_a_bad_program() -> None:
    lib = _lib.load()
    p = _prog([(1, 0, 0, 0)], 1)
    p.ninstr = _site.MAX_SINSTR + 1
    assert lib.plx_site_compile(ctypes.byref(_desc(p)), CSRC, b"gfx950", None) != 0
    p.ninstr = 1
    assert lib.plx_site_compile(ctypes.byref(_desc(p, kind=9)), CSRC, b"gfx950", None) != 0
    with pytest.raises(Exception):
        _lib.check(lib.plx_site_compile(None, CSRC, b"gfx950", None), "plx_site_compile")


def test_forward_prune_compiles() -> None:
    """The fused forward + PruneConn kernel (plx_forward_prune_compile) for a
    traced hash predicate, under every monoid, with the id arrays the fused
    forward passes; a batched or non-EDGE program and an unknown monoid are
    refused."""

    class HashPrune(px.PruneConn):
        def predicate(self, u, c, cid, g):
            h = c[px.FROM_ID, cid] * jnp.int32(7) + c[px.TO_ID, cid] * jnp.int32(13) + g["step"]
            return (h % jnp.int32(1048573)) == jnp.int32(0)

    udt = {"activation": np.dtype(np.float32), "level": np.dtype(np.int32)}
    cdt = {"from_id": np.dtype(np.int32), "to_id": np.dtype(np.int32), "weight": np.dtype(np.float32)}
    p = _traced(_site.trace_predicate(HashPrune(), udt, cdt, {"step": np.int32(0)}))
    lib = _lib.load()
    for m in (0, 1, 2, 3):  # PLX_MONOID_SUM, _PROD, _MAX, _MIN
        rc = lib.plx_forward_prune_compile(ctypes.byref(_desc(p, ids=True)), m, CSRC, b"gfx950", None)
        assert rc == 0, lib.plx_last_error().decode()[:3000]
    assert lib.plx_forward_prune_compile(ctypes.byref(_desc(p, ids=True)), 9, CSRC, b"gfx950", None) != 0
    assert lib.plx_forward_prune_compile(ctypes.byref(_desc(p, kind=0)), 0, CSRC, b"gfx950", None) != 0
    assert lib.plx_forward_prune_compile(ctypes.byref(_desc(p, batch=4)), 0, CSRC, b"gfx950", None) != 0
