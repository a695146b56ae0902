"""Compiled site programs on the device: the growth, pruning and structural
tests of test_gpu_growth.py and test_gpu_structural_step.py run again with
every site program compiled to its own kernel (plx_site_compile), against
the same oracle, bit for bit. The compiled kernel runs the interpreter's
instructions with literal operands, so both paths give the same bits."""

from __future__ import annotations

import pytest

import plastax_amd.grow as grow
from test_gpu_growth import (  # noqa: F401 -- collected here with compiled site programs
    test_claim_pipeline_golden_on_device,
    test_claim_topological_golden_on_device,
    test_normal_draws_in_proposals_match_oracle,
    test_propose_golden_on_device,
    test_prune_conn_matches_oracle,
    test_random_propose_matches_oracle,
    test_random_score_matches_oracle,
    test_random_score_pipeline_matches_oracle,
    test_score_golden_on_device,
)
from test_gpu_structural_step import (  # noqa: F401
    test_dynamic_sparse_mlp_prune_and_regrow_bit_exact,
    test_growing_reservoir_propose_and_prune_bit_exact,
    test_set_proposer_returning_proposals_bit_exact,
)

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _compiled_sites(monkeypatch):
    monkeypatch.setattr(grow, "COMPILE_SITES", "always")


def test_integer_division_and_modulo_at_their_edges(oracle) -> None:
    """jnp's floor `//` and `%` on int32 (divisor 0 and -1, INT32_MIN,
    signs) from a unit program, 2^18 + 5 sites so the default policy
    compiles it too: the compiled kernel (selects) and the interpreter
    (branches) against the oracle's site interpreter, bit for bit."""
    import numpy as np
    import torch

    import plastax_amd as px
    import plastax_amd.numpy as jnp
    from oracle import growth as og
    from plastax_amd import _site

    A = px.FieldSpec("a", np.int32, 0)
    Bf = px.FieldSpec("b", np.int32, 1)

    class DivMod(px.UpdateUnit):
        def update(self, u, i, g):
            a, b = u[A, i], u[Bf, i]
            return px.UnitWrite.of((A, a // b), (Bf, a % b))

    n = (1 << 18) + 5
    rng = np.random.default_rng(11)
    special = np.int32([0, 1, -1, 2, -2, 7, -7, 2**31 - 1, -(2**31), -(2**31) + 1, 65536, -65536])
    a = rng.integers(-(2**31), 2**31, n, dtype=np.int64).astype(np.int32)
    b = rng.integers(-(2**31), 2**31, n, dtype=np.int64).astype(np.int32)
    b[::3] >>= rng.integers(0, 31, b[::3].size).astype(np.int32)  # small divisors too
    m = special.size
    a[: m * m] = np.repeat(special, m)
    b[: m * m] = np.tile(special, m)
    b[m * m :: 7] = special[rng.integers(0, m, b[m * m :: 7].size)]
    units = {"a": a, "b": b}
    dtypes = {"a": np.dtype(np.int32), "b": np.dtype(np.int32)}
    prog, names = _site.trace_update_unit(DivMod(), dtypes, None)
    assert names == ["a", "b"]
    want = og.site_eval(prog, n, {"i": np.arange(n, dtype=np.int32)}, units, None)
    dev = torch.device("cuda", 0)
    ucols = {k: torch.from_numpy(v).to(dev) for k, v in units.items()}
    from plastax_amd.step import _stream

    for policy in ("always", "never"):
        grow.COMPILE_SITES = policy
        k = grow.Kernels(dev, _stream(dev))
        outs = [torch.empty(n, dtype=torch.int32, device=dev) for _ in names]
        k.site_eval(prog, ucols, None, n=n, kind=0, per=1, num_units=n, outs=outs)
        torch.cuda.synchronize()
        for j, name in enumerate(names):
            got = outs[j].cpu().numpy()
            exp = np.asarray(want[j]).astype(np.int32)
            bad = np.flatnonzero(got != exp)
            assert bad.size == 0, (f"{policy}: {name} at a={a[bad[0]]} b={b[bad[0]]}: "
                                   f"{got[bad[0]]} vs {exp[bad[0]]}")
        print(f"int32 // and % over {n} sites equal ({policy})", flush=True)
