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
