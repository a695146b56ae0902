"""Perturbation study of the elementary functions (CPU only; test
infrastructure, like the rest of oracle/).

The reference computes tanh / exp / log with XLA's own float32 kernels, which
cannot run here (no jax), so parity with its trajectory at that boundary is
unpinned. This study bounds how much that boundary can matter: it runs the
oracle twice on the same net and inputs, once with its Cephes restatement of
exp / log / tanh (bit-identical to the device) and once with the C library's
functions (libplastax_oracle_libm.so; glibc's float32 functions are within
about 1 ulp of the true values, as XLA's are within a few), and reports how
far the two trajectories drift apart.

    python -m oracle.perturb [--steps 1000]   (or python oracle/perturb.py)

Prints, at steps 1, 10, 100 and the last, per configuration: the largest
absolute and relative difference over every float unit and connection
column (relative over entries with |value| > 1e-6), and the share of entries
outside rel 1e-5 / abs 1e-6.
"""

from __future__ import annotations

import argparse
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[1]
# (run as a script, this directory comes first on the path and shadows the
# package of the same name)
sys.path = [q for q in sys.path if pathlib.Path(q or ".").resolve() != ROOT / "oracle"]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import plastax_amd as px  # noqa: E402
import plastax_amd.numpy as jnp  # noqa: E402
from oracle import oracle as ox  # noqa: E402
from plastax_amd import synth  # noqa: E402
from plastax_amd._plan import compile_plan  # noqa: E402
from plastax_amd.state import column_to_numpy  # noqa: E402

GRAD = px.FieldSpec.float32("grad_pre_act")
LOSSG = px.FieldSpec.float32("loss_grad")


class Tanh(px.ForwardPass):
    combine = px.monoid.sum_

    def map(self, u, dst, src, c, cid, g):
        return c[px.WEIGHT, cid] * u[px.ACTIVATION, src]

    def apply(self, u, i, g, acc):
        return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc)))


class TanhBack(px.BackwardPass):
    combine = px.monoid.sum_

    def map(self, u, src, dst, c, cid, g):
        return c[px.WEIGHT, cid] * u[GRAD, dst]

    def apply(self, u, i, g, acc):
        a = u[px.ACTIVATION, i]
        return px.UnitWrite.of((GRAD, (acc + u[LOSSG, i]) * (jnp.float32(1.0) - a * a)))


class Mse(px.Loss):
    seed_field = LOSSG

    def calculate_loss(self, u, outputs, targets, g):
        d = u.gather(px.ACTIVATION, outputs) - targets
        return jnp.sum(jnp.float32(0.5) * d * d), d


def make_net(opt, propagation):
    return type("PerturbNet", (px.Network,), dict(
        forward_pass=Tanh(), backward_pass=TanhBack(), loss=Mse(), update_conn=opt.update_conn(),
        extra_unit_fields=(GRAD, LOSSG), extra_conn_fields=tuple(opt.state_fields), propagation=propagation))


def configs(steps: int):
    """(name, net, edges, inputs(k) -> (x, target))."""
    e1 = synth.c1_pipeline(0)
    a = synth.c1_target(0)
    x1 = np.random.default_rng(7).standard_normal((steps, 32)).astype(np.float32)
    yield ("C1 (pipeline, SGD 1e-2)", make_net(px.optim.sgd(1e-2, GRAD), px.Propagation.PIPELINE), e1,
           lambda k: (x1[k], (a @ x1[k]).astype(np.float32)))
    e2 = synth.c2_topological(seed=5, scale=64)
    w = e2.input_ids.size
    sign, perm = synth.c2_target(5, w)
    x2 = np.random.default_rng(13).standard_normal((steps, w)).astype(np.float32)
    yield ("C2 generator at 1/64 width (Adam 1e-3)",
           make_net(px.optim.adam(1e-3, GRAD), px.Propagation.TOPOLOGICAL), e2,
           lambda k: (x2[k], (sign * x2[k][perm]).astype(np.float32)))


def divergence(a: dict, b: dict) -> tuple[float, float, float]:
    """Max abs, max rel (|ref| > 1e-6) and the share outside rel 1e-5 / abs 1e-6."""
    mabs = mrel = 0.0
    bad = total = 0
    for k, ref in b.items():
        if ref.dtype != np.float32:
            continue
        got = a[k]
        d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
        r = np.abs(ref.astype(np.float64))
        fin = np.isfinite(d)
        mabs = max(mabs, float(d[fin].max(initial=0.0)))
        big = fin & (r > 1e-6)
        if big.any():
            mrel = max(mrel, float((d[big] / r[big]).max()))
        bad += int(((d > 1e-6) & (d > 1e-5 * r)).sum())
        total += ref.size
    return mabs, mrel, bad / max(total, 1)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=1000)
    args = ap.parse_args()
    ox.build()
    libm = ox.load_variant(ox.HERE / "libplastax_oracle_libm.so")
    checks = sorted({1, 10, 100, args.steps} & set(range(1, args.steps + 1)))
    for name, net, e, inputs in configs(args.steps):
        static, state = px.NetworkBuilder.from_edges(
            net, e.num_units, e.src, e.dst, weights=e.weight, input_ids=e.input_ids,
            output_ids=e.output_ids, globals_=None, device="cpu")
        specs = {s.name: s for s in static.conn_fields}
        units = {s.name: column_to_numpy(state.units[s.name], s).copy() for s in static.unit_fields}
        conns = [{n: column_to_numpy(bk[n], specs[n]).copy() for n in specs} for bk in state.conns]
        plan = compile_plan(net, static)
        runs = []
        for lib in (None, libm):
            o = ox.OracleNet(static, {k: v.copy() for k, v in units.items()},
                             [{k: v.copy() for k, v in bk.items()} for bk in conns], plan)
            if lib is not None:
                o.lib = lib
            runs.append(o)
        print(f"{name}: {int(e.src.size)} edges", flush=True)
        print("  step   loss(Cephes)      loss(libm)        max abs     max rel     outside rel1e-5/abs1e-6")
        for k in range(1, args.steps + 1):
            x, t = inputs(k - 1)
            la, lb = runs[0].step(x, t), runs[1].step(x, t)
            if k in checks:
                ca = {**runs[1].units, **{f"{b}/{n}": v for b, bk in enumerate(runs[1].conns) for n, v in bk.items()}}
                cb = {**runs[0].units, **{f"{b}/{n}": v for b, bk in enumerate(runs[0].conns) for n, v in bk.items()}}
                mabs, mrel, share = divergence(ca, cb)
                print(f"  {k:5d}  {float(la):.9g}  {float(lb):.9g}  {mabs:10.3e}  {mrel:10.3e}  {share:.3e}",
                      flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
