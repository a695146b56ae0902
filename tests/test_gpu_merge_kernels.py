"""plx_merge_index / plx_merge_gather / plx_remap_i32 / plx_remap_merged /
plx_claimed_split through the C ABI against numpy: two sorted id lists merged by (key1, key2)
(a first on equal keys), the order and both maps; a multi-column gather from the two sides;
short b (keys staged in LDS) and long b (searched in global memory), empty
sides, ties across the sides; a claim's slot list split by bucket."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from plastax_amd import _lib

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _t(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _side(side, ids, k1, k2, out_map, limit):
    side.n, side.id_limit = int(ids.numel()), int(limit)
    side.ids, side.key1 = ids.data_ptr(), k1.data_ptr()
    side.key2 = None if k2 is None else k2.data_ptr()
    side.map = None if out_map is None else out_map.data_ptr()


def _case(rng, na: int, nb: int, limit: int, nkeys: int, ties: bool):
    """Ids sorted by (key1, key2 = slot-like unique values)."""
    key1 = rng.integers(0, nkeys, limit).astype(np.int32)
    key2 = rng.permutation(limit).astype(np.int32)
    ids = rng.permutation(limit)
    a_ids = np.sort(ids[:na])
    b_ids = np.sort(ids[na : na + nb])
    a_ids = a_ids[np.lexsort((key2[a_ids], key1[a_ids]))].astype(np.int32)
    b_key2 = key2.copy()
    if ties and na and nb:  # b's first element takes a's first element's key
        b_key2[b_ids[0]] = key2[a_ids[0]]
        key1_b = key1.copy()
        key1_b[b_ids[0]] = key1[a_ids[0]]
    else:
        key1_b = key1
    b_ids = b_ids[np.lexsort((b_key2[b_ids], key1_b[b_ids]))].astype(np.int32)
    return key1, key2, key1_b, b_key2, a_ids, b_ids


@pytest.mark.parametrize(("na", "nb"), [(5000, 37), (5000, 3000), (0, 100), (4000, 0), (1, 1), (300, 2048),
                                        (257, 2049)])
@pytest.mark.parametrize("ties", [False, True])
def test_merge_index_and_gather(na: int, nb: int, ties: bool) -> None:
    lib = _lib.load()
    rng = np.random.default_rng(na * 7 + nb + ties)
    limit = na + nb + 64
    k1, k2, k1b, k2b, a_ids, b_ids = _case(rng, na, nb, limit, max(4, limit // 9), ties)
    # expected: a first where keys are equal
    keys = [((int(k1[i]) & 0xFFFFFFFF) << 32 | (int(k2[i]) & 0xFFFFFFFF), 0, r, int(i)) for r, i in enumerate(a_ids)]
    keys += [((int(k1b[i]) & 0xFFFFFFFF) << 32 | (int(k2b[i]) & 0xFFFFFFFF), 1, r, int(i))
             for r, i in enumerate(b_ids)]
    keys.sort()
    want_order = np.asarray([i if side == 0 else -1 - r for _, side, r, i in keys], dtype=np.int32)
    n = na + nb
    order = torch.full((max(n, 1),), 7777, dtype=torch.int32, device=DEV)
    map_a = torch.full((limit,), -1, dtype=torch.int32, device=DEV)
    map_b = torch.full((limit,), -1, dtype=torch.int32, device=DEV)
    ta, tb = _t(a_ids), _t(b_ids)
    m = _lib.plx_merge_desc()
    _side(m.a, ta, _t(k1), _t(k2), map_a, limit)
    _side(m.b, tb, _t(k1b), _t(k2b), map_b, limit)
    m.offset, m.order = 100, order.data_ptr()
    assert lib.plx_merge_index(m, None) == 0, lib.plx_last_error()
    torch.cuda.synchronize()
    assert np.array_equal(order.cpu().numpy()[:n], want_order)
    ma, mb = map_a.cpu().numpy(), map_b.cpu().numpy()
    for r, (_, side, _, i) in enumerate(keys):
        assert (ma if side == 0 else mb)[i] == r + 100
    # gather: a 4-byte column, a 1-byte column, b's id itself
    if n == 0:
        return
    col_a = rng.standard_normal(limit).astype(np.float32)
    col_b = rng.standard_normal(limit).astype(np.float32)
    u8_a = rng.integers(0, 255, limit).astype(np.uint8)
    u8_b = rng.integers(0, 255, limit).astype(np.uint8)
    outs = [torch.empty(n, dtype=torch.float32, device=DEV), torch.empty(n, dtype=torch.uint8, device=DEV),
            torch.empty(n, dtype=torch.int32, device=DEV)]
    ins = [(_t(col_a), _t(col_b), 4), (_t(u8_a), _t(u8_b), 1), (_t(np.arange(limit, dtype=np.int32)), None, 4)]
    g = _lib.plx_merge_gather_desc()
    g.n, g.order, g.b_ids, g.nb, g.a_limit, g.b_limit = n, order.data_ptr(), tb.data_ptr(), nb, limit, limit
    g.ncols = 3
    for j, ((a, b, nbytes), out) in enumerate(zip(ins, outs)):
        g.cols[j].a, g.cols[j].b = a.data_ptr(), (None if b is None else b.data_ptr())
        g.cols[j].out, g.cols[j].bytes = out.data_ptr(), nbytes
    assert lib.plx_merge_gather(g, None) == 0, lib.plx_last_error()
    torch.cuda.synchronize()
    src_a = want_order >= 0
    ids_all = np.where(src_a, want_order, b_ids[np.where(src_a, 0, -1 - want_order)] if nb else 0)
    assert np.array_equal(outs[0].cpu().numpy(), np.where(src_a, col_a[ids_all], col_b[ids_all]))
    assert np.array_equal(outs[1].cpu().numpy(), np.where(src_a, u8_a[ids_all], u8_b[ids_all]))
    assert np.array_equal(outs[2].cpu().numpy(), ids_all.astype(np.int32))


def test_remap() -> None:
    lib = _lib.load()
    rng = np.random.default_rng(9)
    base, n_map = 1000, 5000
    mp = np.where(rng.random(n_map) < 0.3, -1, rng.integers(0, 10**6, n_map)).astype(np.int32)
    idx = (base + rng.integers(-5, n_map + 5, 20000)).astype(np.int32)
    out = torch.empty(idx.size, dtype=torch.int32, device=DEV)
    live = torch.empty(idx.size, dtype=torch.uint8, device=DEV)
    tm = _t(mp)
    assert lib.plx_remap_i32(idx.size, _t(idx).data_ptr(), base, n_map, tm.data_ptr(), out.data_ptr(),
                             live.data_ptr(), None) == 0
    torch.cuda.synchronize()
    p = idx.astype(np.int64) - base
    want = np.where((p >= 0) & (p < n_map), mp[np.clip(p, 0, n_map - 1)], -1)
    assert np.array_equal(out.cpu().numpy(), want)
    assert np.array_equal(live.cpu().numpy(), (want >= 0).astype(np.uint8))


@pytest.mark.parametrize(("na", "nb", "pad_a", "pad_b"), [(5000, 37, 800, 60), (0, 100, 300, 20), (4000, 0, 5, 9),
                                                          (300, 2048, 1000, 100), (257, 2049, 3, 3000)])
def test_merge_with_device_counts(na: int, nb: int, pad_a: int, pad_b: int) -> None:
    """The sides' counts on the device (n_dev) below their host bounds, the
    id lists holding garbage past the counts: the merge sees only the counted
    elements; the gather with a device output count writes each column's
    fill bits at the ranks from the count to its bound, and the sorted starts
    count only the first n_dev keys."""
    lib = _lib.load()
    rng = np.random.default_rng(na + 3 * nb + pad_a)
    limit = na + nb + 64
    k1, k2, k1b, k2b, a_ids, b_ids = _case(rng, na, nb, limit, max(4, limit // 9), False)
    keys = [((int(k1[i]) & 0xFFFFFFFF) << 32 | (int(k2[i]) & 0xFFFFFFFF), 0, r, int(i)) for r, i in enumerate(a_ids)]
    keys += [((int(k1b[i]) & 0xFFFFFFFF) << 32 | (int(k2b[i]) & 0xFFFFFFFF), 1, r, int(i))
             for r, i in enumerate(b_ids)]
    keys.sort()
    want_order = np.asarray([i if side == 0 else -1 - r for _, side, r, i in keys], dtype=np.int32)
    # garbage ids past the counts (in range, so any read stays in bounds)
    ga = np.concatenate([a_ids, rng.integers(0, limit, pad_a)]).astype(np.int32)
    gb = np.concatenate([b_ids, rng.integers(0, limit, pad_b)]).astype(np.int32)
    bound = ga.size + gb.size
    order = torch.full((max(bound, 1),), 7777, dtype=torch.int32, device=DEV)
    ta, tb = _t(ga), _t(gb)
    na_d, nb_d = _t(np.int32([na])), _t(np.int32([nb]))
    m = _lib.plx_merge_desc()
    _side(m.a, ta, _t(k1), _t(k2), None, limit)
    _side(m.b, tb, _t(k1b), _t(k2b), None, limit)
    m.a.n_dev, m.b.n_dev = na_d.data_ptr(), nb_d.data_ptr()
    m.offset, m.order = 0, order.data_ptr()
    assert lib.plx_merge_index(m, None) == 0, lib.plx_last_error()
    torch.cuda.synchronize()
    n = na + nb
    assert np.array_equal(order.cpu().numpy()[:n], want_order)
    if n:
        col_a = rng.standard_normal(limit).astype(np.float32)
        col_b = rng.standard_normal(limit).astype(np.float32)
        out_f = torch.empty(bound, dtype=torch.float32, device=DEV)
        out_u = torch.empty(bound, dtype=torch.uint8, device=DEV)
        u8 = _t(rng.integers(0, 255, limit).astype(np.uint8))
        g = _lib.plx_merge_gather_desc()
        g.n, g.order, g.b_ids, g.nb, g.a_limit, g.b_limit = bound, order.data_ptr(), tb.data_ptr(), gb.size, limit, limit
        n_d = _t(np.int32([n]))
        g.n_dev = n_d.data_ptr()
        g.ncols = 2
        ta_f, tb_f = _t(col_a), _t(col_b)
        g.cols[0].a, g.cols[0].b, g.cols[0].out, g.cols[0].bytes = ta_f.data_ptr(), tb_f.data_ptr(), out_f.data_ptr(), 4
        g.cols[0].fill = int(np.float32(-2.5).view(np.uint32))
        g.cols[1].a, g.cols[1].b, g.cols[1].out, g.cols[1].bytes = u8.data_ptr(), u8.data_ptr(), out_u.data_ptr(), 1
        g.cols[1].fill = 1
        assert lib.plx_merge_gather(g, None) == 0, lib.plx_last_error()
        torch.cuda.synchronize()
        src_a = want_order >= 0
        ids_all = np.where(src_a, want_order, b_ids[np.where(src_a, 0, -1 - want_order)] if nb else 0)
        got = out_f.cpu().numpy()
        assert np.array_equal(got[:n], np.where(src_a, col_a[ids_all], col_b[ids_all]))
        assert np.all(got[n:] == np.float32(-2.5)) and np.all(out_u.cpu().numpy()[n:] == 1)
    # sorted starts over the first n_dev keys of a list with garbage after them
    keys_s = np.sort(rng.integers(0, 50, max(n, 1))).astype(np.int32)[: max(n, 1)]
    cnt = int(min(n, keys_s.size))
    padded = np.concatenate([keys_s[:cnt], rng.integers(0, 3, 40)]).astype(np.int32)
    start = torch.empty(51, dtype=torch.int32, device=DEV)
    assert lib.plx_sorted_starts(padded.size, _t(np.int32([cnt])).data_ptr(), _t(padded).data_ptr(), 50,
                                 start.data_ptr(), None) == 0
    torch.cuda.synchronize()
    assert np.array_equal(start.cpu().numpy(), np.searchsorted(keys_s[:cnt], np.arange(51), side="left"))


@pytest.mark.parametrize("caps,nlisted,cap,region", [
    ([100, 0, 37, 513], 40, 64, 64),        # an empty bucket, a short list
    ([4096], 4096, 4096, 4096),             # one bucket, the largest list
    ([50, 50, 50], 20, 32, 8),              # a region shorter than a bucket's count
    ([10, 20], 0, 16, 16),                  # nothing claimed
    ([3000, 5000], 100, 128, 128),          # the device count past cap
])
def test_claimed_split(caps, nlisted, cap, region) -> None:
    """plx_claimed_split against numpy: each bucket's listed slots less its
    start, ascending, the first `region` of them, and their count."""
    rng = np.random.default_rng(sum(caps) + nlisted)
    offs = np.concatenate([[0], np.cumsum(caps)]).astype(np.int64)
    total = int(offs[-1])
    listed = rng.choice(total, size=min(nlisted, total), replace=False).astype(np.int32)
    buf = np.full(max(cap, 1), -7, np.int32)
    n_dev = min(nlisted, len(listed))
    buf[: min(n_dev, cap)] = listed[: min(n_dev, cap)]
    if caps == [3000, 5000]:
        n_dev = cap + 50  # appends past cap were never written: only cap entries count
    nb = len(caps)
    out = torch.full((nb, max(region, 1)), -1, dtype=torch.int32, device=DEV)
    counts = torch.full((nb,), -1, dtype=torch.int32, device=DEV)
    lst, nd, offs_t = _t(buf), _t(np.array([n_dev], np.int32)), _t(offs)
    _lib.call("plx_claimed_split", cap, nd.data_ptr(), lst.data_ptr(), nb, offs_t.data_ptr(), region,
              out.data_ptr(), counts.data_ptr(), None)
    torch.cuda.synchronize()
    got_out, got_counts = out.cpu().numpy(), counts.cpu().numpy()
    seen = buf[: min(n_dev, cap)]
    for b in range(nb):
        want = np.sort(seen[(seen >= offs[b]) & (seen < offs[b + 1])] - offs[b])
        assert got_counts[b] == want.size, f"bucket {b}: count"
        k = min(want.size, region)
        assert np.array_equal(got_out[b, :k], want[:k]), f"bucket {b}: slots"
        assert np.all(got_out[b, k:] == -1), f"bucket {b}: wrote past its slots"
    with pytest.raises(_lib.PlxError):
        _lib.call("plx_claimed_split", 4097, nd.data_ptr(), lst.data_ptr(), nb, offs_t.data_ptr(), region,
                  out.data_ptr(), counts.data_ptr(), None)


@pytest.mark.parametrize("m,ndrop,nins", [(5000, 40, 32), (20000, 0, 0), (20000, 3000, 4096), (30000, 5000, 10)])
def test_remap_merged(m: int, ndrop: int, nins: int) -> None:
    """plx_remap_merged against the old-to-new map of the same merge (numpy):
    m old positions, `ndrop` of them dropped, `nins` elements inserted at
    random survivor ranks; list entries at random positions (some outside
    the map). More than PLX_REMAP_LDS_MAX dropped positions take the map."""
    rng = np.random.default_rng(m + ndrop + nins)
    off = 1000
    dropped = np.sort(rng.choice(m, ndrop, replace=False)).astype(np.int32)
    surv = np.setdiff1d(np.arange(m), dropped)
    ranks = np.sort(rng.integers(0, surv.size + 1, nins))  # survivors before each inserted element
    # merged order: survivor s at s + #(ranks <= s); inserted i at ranks[i] + i
    old_to_new = np.full(m, -1, np.int32)
    old_to_new[surv] = np.arange(surv.size) + np.searchsorted(ranks, np.arange(surv.size), side="right") + off
    ins = rng.permutation(max(nins, 1)).astype(np.int32)[:nins]  # slot ids of the inserted elements
    new_pos = np.full(max(nins, 1) + 5, -7, np.int32)
    new_pos[ins] = ranks + np.arange(nins) + off
    n = 70000
    idx = (rng.integers(-50, m + 50, n) + off).astype(np.int32)
    want = np.full(n, -1, np.int32)
    inside = (idx - off >= 0) & (idx - off < m)
    want[inside] = old_to_new[idx[inside] - off]
    out = torch.empty(n, dtype=torch.int32, device=DEV)
    live = torch.empty(n, dtype=torch.uint8, device=DEV)
    t_idx, t_map, t_drop = _t(idx), _t(old_to_new), _t(dropped if ndrop else np.zeros(1, np.int32))
    t_ins, t_new = _t(ins if nins else np.zeros(1, np.int32)), _t(new_pos)
    nd, ni = _t(np.array([ndrop], np.int32)), _t(np.array([nins], np.int32))
    _lib.call("plx_remap_merged", n, t_idx.data_ptr(), off, m, t_map.data_ptr(), t_drop.data_ptr(), nd.data_ptr(),
              t_ins.data_ptr(), ni.data_ptr(), max(nins, 1), t_new.data_ptr(), out.data_ptr(), live.data_ptr(), None)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want)
    assert np.array_equal(live.cpu().numpy(), (want >= 0).astype(np.uint8))
