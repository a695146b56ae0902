"""The CPU oracle against the reference's golden vectors (CPU only).

Goldens are the reference's own fixtures (tests/golden/*.json, emitted by
scripts/parity/emit.py and consumed by tests/test_parity_goldens.py:245-350
in the reference). Every value in them is dyadic, so float32 arithmetic on
them is exact and the comparison is exact. The policies are traced by the
framework exactly as the device path traces them.
"""

from __future__ import annotations

import numpy as np
import pytest

import nets


def test_passes_relu_topological_matches_golden_exactly(oracle) -> None:
    doc = nets.load_golden("passes_relu_topological.json")
    static, state = nets.build_golden(nets.ReluMlpNet, doc)
    o = nets.oracle_for(oracle, nets.ReluMlpNet, static, state)
    for i, s in enumerate(doc["steps"]):
        loss = o.step(s["inputs"], s["targets"])
        acts = o.units["activation"].tolist()
        grads = o.units["grad_pre_act"].tolist()
        assert acts == s["expect"]["activations"], f"step {i} activations"
        assert grads == s["expect"]["grad_pre_act"], f"step {i} grads"
        assert float(loss) == s["expect"]["loss"], f"step {i} loss"


def test_passes_relu_pipeline_matches_golden_exactly(oracle) -> None:
    doc = nets.load_golden("passes_relu_pipeline.json")
    static, state = nets.build_golden(nets.ReluPipelineNet, doc)
    o = nets.oracle_for(oracle, nets.ReluPipelineNet, static, state)
    for i, s in enumerate(doc["steps"]):
        o.step(s["inputs"])
        assert o.units["activation"].tolist() == s["expect"]["activations"], f"step {i}"


LOSS_GOLDENS = [
    "loss_softmax_ce_large_logits",
    "loss_softmax_ce_negative_logits",
    "loss_softmax_ce_one_hot",
    "loss_softmax_ce_soft_targets",
    "loss_softmax_ce_tied_max",
]


@pytest.mark.parametrize("name", LOSS_GOLDENS)
def test_softmax_ce_matches_golden_exactly(oracle, name: str) -> None:
    doc = nets.load_golden(f"{name}.json")
    assert doc["rules"] == {
        "loss": "softmax_ce_v1",
        "forward": "linear_v1",
        "weights": "identity_weight_v1",
    }
    static, state = nets.build_golden(nets.SoftmaxNet, doc)
    out = list(static.output_ids)
    o = nets.oracle_for(oracle, nets.SoftmaxNet, static, state)
    for i, s in enumerate(doc["steps"]):
        loss = o.step(s["inputs"], s["targets"])
        assert o.units["activation"][out].tolist() == s["expect"]["activations"], f"step {i}"
        assert o.units["loss_grad"][out].tolist() == s["expect"]["seed"], f"step {i} seed"
        assert float(loss) == s["expect"]["loss"], f"step {i} loss"


def test_golden_fixtures_are_all_consumed() -> None:
    """Every golden fixture copied into tests/golden has a consumer here."""
    import growth_cases

    names = {p.stem for p in nets.GOLDEN.glob("*.json")}
    growth = {p.stem for p in nets.GOLDEN.glob("grow_*.json")}
    assert growth == set(growth_cases.names(lambda d: True))  # test_growth_oracle.py
    units = {p.stem for p in nets.GOLDEN.glob("unit_*.json")}  # test_unit_oracle.py
    consumed = {"passes_relu_topological", "passes_relu_pipeline", *LOSS_GOLDENS, *growth, *units}
    assert names == consumed


def test_pipeline_crosses_one_connection_per_step(oracle) -> None:
    """A PIPELINE net needs L steps to carry an input to level L, and then
    matches the TOPOLOGICAL forward (reference test_forward_topo.py:148-196)."""
    doc = nets.load_golden("passes_relu_topological.json")
    st_topo, s_topo = nets.build_golden(nets.ReluMlpNet, doc)
    st_pipe, s_pipe = nets.build_golden(nets.ReluPipelineNet, doc)
    topo = nets.oracle_for(oracle, nets.ReluMlpNet, st_topo, s_topo)
    pipe = nets.oracle_for(oracle, nets.ReluPipelineNet, st_pipe, s_pipe)
    x = [0.75, -0.25]
    topo.step(x, [0.0, 0.0])
    for _ in range(2):  # two connection hops to the output level
        pipe.step(x)
    assert pipe.units["activation"].tolist() == topo.units["activation"].tolist()
