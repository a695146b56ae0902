"""The C-ABI library loads and exports what include/plastax_hip.h declares
(CPU only: no kernel is launched)."""

from __future__ import annotations

import ctypes
import pathlib
import re

import pytest

from plastax_amd import _lib

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "plastax_hip.h"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"PLX_EXPORT\s+[\w\s\*]+?\b(plx_\w+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from plastax_amd import build

        build.build()
    return _lib.load()


def test_header_declares_the_bound_entry_points() -> None:
    assert declared_symbols() == set(_lib.EXPORTED)


def test_library_exports_every_declared_symbol(lib) -> None:
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_descriptor_layouts_match_the_header(lib) -> None:
    n = len(_lib.STRUCTS)
    out = (ctypes.c_int64 * n)()
    assert lib.plx_struct_sizes(out, n) == n == 20
    assert list(out) == [ctypes.sizeof(s) for s in _lib.STRUCTS]
    assert lib.plx_abi_version() == _lib.ABI_VERSION


def test_argument_errors_are_reported_not_raised(lib) -> None:
    """Validation runs before any HIP call, so it is testable without a GPU."""
    rc = lib.plx_forward_bucket(None, None)
    assert rc == 1
    assert b"null descriptor" in lib.plx_last_error()
    d = _lib.plx_update_desc()
    d.n = 6
    assert lib.plx_update_conn(d, None) == 1
    assert b"multiple of 4" in lib.plx_last_error()
    assert lib.plx_fill_f32(-1, 0.0, None, None) == 1
    # zero-sized work is a no-op success
    assert lib.plx_fill_f32(0, 0.0, None, None) == 0
    # the structural entry points validate before launching too
    assert lib.plx_site_eval(None, None) == 1
    sd = _lib.plx_site_desc()
    sd.n, sd.num_units, sd.kind = 4, 8, 9
    sd.prog.ninstr = 0
    assert lib.plx_site_eval(sd, None) == 1
    assert b"unknown site kind" in lib.plx_last_error()
    sd.kind, sd.prog.ninstr = 0, 1
    sd.prog.code[0], sd.prog.code[1], sd.prog.code[2] = 3, 0, 0  # LDU of an unset field
    assert lib.plx_site_eval(sd, None) == 1
    assert b"bad program" in lib.plx_last_error()
    assert lib.plx_compact(-1, None, 0, None, None, None, None, None) == 1
    assert lib.plx_compact(0, None, 0, None, None, None, None, None) == 1  # count is required
    srt = _lib.plx_sort_desc()
    srt.n_max, srt.nkeys = 10, 7
    assert lib.plx_sort(srt, None) == 1
    assert lib.plx_scratch_ints(4096) >= 256 + 2
    cd = _lib.plx_grow_claim_desc()
    cd.n_max = 0
    assert lib.plx_grow_claim(cd, None) == 0
    # batched entry points
    fd = _lib.plx_forward_desc()
    fd.nrows = 3
    assert lib.plx_forward_batch(fd, 0, None) == 1
    assert b"batch must be >= 1" in lib.plx_last_error()
    assert lib.plx_forward_batch(fd, 4, None) == 1
    assert b"null column" in lib.plx_last_error()
    bd = _lib.plx_bwd_batch_desc()
    bd.batch, bd.nrows = 2, 0
    assert lib.plx_backward_batch(bd, None) == 0
    ud = _lib.plx_update_desc()
    ud.n = 5
    assert lib.plx_update_batch(ud, 2, None) == 1
    assert b"null column" in lib.plx_last_error()
    assert lib.plx_reduce_batch(4, 2, 0, 1, None, None, None) == 1
    assert b"MEAN needs a float32" in lib.plx_last_error()
    assert lib.plx_reduce_batch(4, 2, 1, 2, None, None, None) == 1
    assert b"FIRST only" in lib.plx_last_error()
    assert lib.plx_batch_mean(0, None, None, None) == 1


def test_batch_tile_limits_match_the_layout(lib) -> None:
    """The batched-update kernel's tile limits, queried through the ABI,
    are the ones plastax_amd._layout.batch_tiles builds for."""
    from plastax_amd import _layout

    rows, edges = ctypes.c_int32(), ctypes.c_int32()
    assert lib.plx_batch_tile_limits(ctypes.byref(rows), ctypes.byref(edges)) == 0
    assert (rows.value, edges.value) == (_layout.BATCH_TILE_UNITS, _layout.BATCH_TILE_EDGES)
    assert lib.plx_batch_tile_limits(None, None) != 0
