"""plx_compact_noalloc (the allocation-free ordered compaction) against
plx_compact, through the C ABI: two calls in a row, the second smaller, on
every flag mode, with and without a device-side live count."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from plastax_amd import _lib

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
MAX_N = 1 << 26


def _flags(rng: np.random.Generator, n: int, mode: int) -> torch.Tensor:
    if mode in (0, 1):
        return torch.from_numpy((rng.random(n) < 0.37).astype(np.uint8)).to(DEV)
    if mode == 2:
        v = rng.standard_normal(n).astype(np.float32)
        v[rng.random(n) < 0.3] = np.inf
        v[rng.random(n) < 0.1] = np.nan
        return torch.from_numpy(v).to(DEV)
    return torch.from_numpy(rng.integers(-2, 3, n).astype(np.int32)).to(DEV)


def _both(n: int, mode: int, flags: torch.Tensor, n_dev: torch.Tensor | None):
    stream = torch.cuda.current_stream(DEV).cuda_stream
    outs = []
    for noalloc in (False, True):
        out = torch.full((max(n, 1),), -7, dtype=torch.int32, device=DEV)
        count = torch.full((1,), -7, dtype=torch.int32, device=DEV)
        nd = n_dev.data_ptr() if n_dev is not None else None
        if noalloc:
            _lib.call("plx_compact_noalloc", n, nd, mode, flags.data_ptr(), out.data_ptr(), count.data_ptr(), stream)
        else:
            scratch = torch.empty(max(int(_lib.load().plx_scratch_ints(n)), 1), dtype=torch.int32, device=DEV)
            _lib.call("plx_compact", n, nd, mode, flags.data_ptr(), out.data_ptr(), count.data_ptr(),
                      scratch.data_ptr(), stream)
        torch.cuda.synchronize()
        c = int(count.item())
        outs.append((c, out[:c].cpu().numpy()))
    return outs


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_noalloc_compaction_equals_plx_compact(mode: int) -> None:
    rng = np.random.default_rng(40 + mode)
    for n in (3_000_001, 70_003):  # the second call is smaller: stale chunk sums must not leak
        flags = _flags(rng, n, mode)
        (c0, o0), (c1, o1) = _both(n, mode, flags, None)
        print(f"noalloc compaction mode {mode} n {n}: {c1} kept", flush=True)
        assert c0 == c1 and np.array_equal(o0, o1)
        f = flags.cpu().numpy()
        want = {0: f != 0, 1: f == 0, 2: np.isfinite(f) if mode == 2 else None, 3: f != 0}[mode]
        assert np.array_equal(o1, np.flatnonzero(want).astype(np.int32))


def test_noalloc_compaction_with_a_device_count() -> None:
    rng = np.random.default_rng(50)
    n = 1_000_000
    flags = _flags(rng, n, 0)
    for live in (654_321, 4_097):
        n_dev = torch.tensor([live], dtype=torch.int32, device=DEV)
        (c0, o0), (c1, o1) = _both(n, 0, flags, n_dev)
        assert c0 == c1 and np.array_equal(o0, o1)
        assert np.array_equal(o1, np.flatnonzero(flags.cpu().numpy()[:live] != 0).astype(np.int32))


def test_noalloc_compaction_at_its_maximum_size_and_beyond() -> None:
    """n = PLX_COMPACT_NOALLOC_MAX_N uses every chunk sum of the array; one
    more is refused before any launch."""
    flags = torch.zeros(MAX_N, dtype=torch.uint8, device=DEV)
    flags[::1000] = 1
    flags[-1] = 1
    (c0, o0), (c1, o1) = _both(MAX_N, 0, flags, None)
    assert c0 == c1 == (MAX_N - 1) // 1000 + 2 and np.array_equal(o0, o1)
    lib = _lib.load()
    out = torch.empty(1, dtype=torch.int32, device=DEV)
    rc = lib.plx_compact_noalloc(MAX_N + 1, None, 0, ctypes.c_void_p(flags.data_ptr()),
                                 ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(out.data_ptr()), None)
    assert rc != 0 and b"PLX_COMPACT_NOALLOC_MAX_N" in lib.plx_last_error()
