"""The reference's free-slot claim churn (tests/test_growth_claim.py:1-322):
layered nets, a hashed PruneConn killing about rate/256 of the live edges per
step, and hashed growth (global proposals with coarse, tied scores and a
vetoed slice, or a hash-scored grid) refilling them, for 24 steps. The
reference pins the sha256 of the final logical arena (every column of every
bucket by name, then `needs_resort` and the per-step overflow bytes) in
`_GOLDEN` (`:315-321`); weights are small integers, so the digests do not
depend on float rounding. The policies below are the same integer programs,
written against this package's numpy shim.
"""

from __future__ import annotations

import hashlib

import numpy as np

import plastax_amd as px
import plastax_amd.numpy as jnp

AGE = px.FieldSpec.int32("test/age")  # written by init
TRACE = px.FieldSpec.float32("test/trace", default=1.5)  # left at its default
STEPS = 24


def _mix(x):
    """lowbias32 (test_growth_claim.py:36-43)."""
    x = x.astype(jnp.uint32)
    x = x ^ (x >> 16)
    x = x * jnp.uint32(0x7FEB352D)
    x = x ^ (x >> 15)
    x = x * jnp.uint32(0x846CA68B)
    return x ^ (x >> 16)


def _h(*parts):
    acc = jnp.uint32(0x9E3779B9)
    for p in parts:
        acc = _mix(acc ^ jnp.asarray(p).astype(jnp.uint32))
    return acc


class _Forward(px.ForwardPass):
    combine = px.monoid.sum_

    def map(self, u, dst, src, c, cid, g):
        return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, acc))


class _HashPrune(px.PruneConn):
    def __init__(self, rate: int) -> None:
        self.rate = rate

    def predicate(self, u, c, cid, g):
        h = _h(c[px.FROM_ID, cid], c[px.TO_ID, cid], g["t"], jnp.uint32(7))
        return (h & jnp.uint32(255)) < jnp.uint32(self.rate)


def _init(src, dst, g):
    weight = ((src * 3 + dst) % 17).astype(jnp.float32) - 8.0
    return px.ConnWrite.of((px.WEIGHT, weight), (AGE, g["t"] + src))


class _HashProposals(px.ProposeAddConn):
    def __init__(self, num_units: int, num_proposals: int, max_new_per_level: int, dedupe: bool) -> None:
        self.num_units = num_units
        self.proposer = "global"
        self.proposals_per_proposer = num_proposals
        self.max_new_per_level = max_new_per_level
        self.dedupe_live = dedupe
        self.dedupe_step = dedupe

    def propose(self, u, j, g, rng):
        h = _h(j, g["t"], jnp.uint32(11))
        src = (h % jnp.uint32(self.num_units)).astype(jnp.int32)
        h2 = _h(h, jnp.uint32(13))
        dst = (h2 % jnp.uint32(self.num_units)).astype(jnp.int32)
        score = ((h2 >> 8) & jnp.uint32(7)).astype(jnp.float32)
        veto = (h >> 24) < jnp.uint32(40)
        return src, dst, jnp.where(veto, -jnp.inf, score)

    def init(self, u, src, dst, g):
        return _init(src, dst, g)


class _HashGrid(px.ScoreAddConn):
    dedupe_live = True

    def __init__(self, max_new_per_level: int) -> None:
        self.max_new_per_level = max_new_per_level

    def score(self, u, src, dst, g):
        h = _h(src, dst, g["t"], jnp.uint32(17))
        score = (h & jnp.uint32(15)).astype(jnp.float32)
        return jnp.where((h >> 28) < jnp.uint32(3), -jnp.inf, score)

    def init(self, u, src, dst, g):
        return _init(src, dst, g)


class _Tick(px.ResetGlobal):
    def reset(self, g):
        return {"t": g["t"] + jnp.int32(1)}


# test_growth_claim.py:158-230
CONFIGS: dict[str, dict] = {
    "propose_overflow": dict(widths=(12, 16, 16, 8), density=0.5, rate=48, grow="propose",
                             proposals=128, k=128, dedupe=False, headroom=0.02, align=None),
    "propose_dedupe": dict(widths=(12, 16, 16, 8), density=0.5, rate=48, grow="propose",
                           proposals=160, k=48, dedupe=True, headroom=0.1, align=None),
    "propose_small_claim": dict(widths=(96, 128, 64), density=0.6, rate=4, grow="propose",
                                proposals=24, k=4, dedupe=False, headroom=0.05, align=256),
    "propose_window2": dict(widths=(10, 9, 11, 7), density=0.6, rate=40, grow="propose",
                            proposals=48, k=48, dedupe=False, headroom=0.0, align=7, max_level_gap=2),
    "grid": dict(widths=(8, 12, 6), density=0.4, rate=80, grow="grid", k=20, headroom=0.05, align=None),
}

# The reference's pinned final digests (test_growth_claim.py:315-321).
GOLDEN: dict[str, str] = {
    "grid": "4e8864fe12526877",
    "propose_dedupe": "e9b8e9998f5449b8",
    "propose_overflow": "7b3e8de90e4863c4",
    "propose_small_claim": "84b5c49d0d202d72",
    "propose_window2": "54a96de099f5a4b1",
}


def build(name: str, device: str):
    """The config's net, static and state (test_growth_claim.py:233-281)."""
    cfg = CONFIGS[name]
    rng = np.random.default_rng(0)
    widths = cfg["widths"]
    offsets = np.concatenate([[0], np.cumsum(widths)])
    num_units = int(offsets[-1])
    frm, to = [], []
    for layer in range(len(widths) - 1):
        a = np.arange(offsets[layer], offsets[layer + 1])
        b = np.arange(offsets[layer + 1], offsets[layer + 2])
        src, dst = np.meshgrid(a, b, indexing="ij")
        keep = rng.random(src.shape) < cfg["density"]
        frm.append(src[keep])
        to.append(dst[keep])
    from_ids = np.concatenate(frm).astype(np.int32)
    to_ids = np.concatenate(to).astype(np.int32)
    if cfg["grow"] == "propose":
        policy = _HashProposals(num_units, cfg["proposals"], cfg["k"], cfg["dedupe"])
    else:
        policy = _HashGrid(cfg["k"])
    policy.max_level_gap = cfg.get("max_level_gap", 1)
    prune = _HashPrune(cfg["rate"])

    class Net(px.Network):
        forward_pass = _Forward()
        prune_conn = prune
        add_conn = policy
        reset_global = _Tick()
        extra_conn_fields = (AGE, TRACE)
        propagation = px.Propagation.TOPOLOGICAL

    static, state = px.NetworkBuilder.from_edges(
        Net, num_units, from_ids, to_ids, weights=np.ones(from_ids.size, np.float32),
        input_ids=list(range(widths[0])), output_ids=list(range(int(offsets[-2]), num_units)),
        globals_={"t": np.int32(0)}, capacity_headroom=cfg["headroom"], capacity_align=cfg["align"],
        device=device)
    return Net, static, state


def digest(conns, needs_resort: bool, overflows: list[bool]) -> str:
    """test_growth_claim.py:273-281: columns by name per bucket, then the
    resort flag and the overflow bytes."""
    h = hashlib.sha256()
    for bucket in conns:
        for name in sorted(bucket):
            col = bucket[name]
            arr = col.detach().cpu().numpy() if hasattr(col, "detach") else np.asarray(col)
            h.update(name.encode())
            h.update(np.ascontiguousarray(arr).tobytes())
    h.update(bytes([bool(needs_resort)]))
    h.update(bytes(overflows))
    return h.hexdigest()[:16]
