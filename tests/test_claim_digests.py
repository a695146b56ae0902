"""The reference's claim churn digests (test_growth_claim.py:283-344): 24
steps of hashed PruneConn + growth per config, the whole logical arena and
the flags hashed at the end. The oracle must reproduce the reference's pinned
digests; the device path (GPU tests) must reproduce them too, and agree with
the oracle's flags at every step."""

from __future__ import annotations

import numpy as np
import pytest

import claim_cases as cc
import nets


def _oracle_run(ox, name: str):
    net, static, state = cc.build(name, "cpu")
    o = nets.oracle_for(ox, net, static, state)
    o.tail_start, o.needs_resort = int(state.tail_start), bool(state.needs_resort)
    x = np.ones(len(static.input_ids), np.float32)
    flags, overflows = [], []
    for _ in range(cc.STEPS):
        o.step(x, None)
        overflows.append(bool(o.overflow))
        flags.append((o.grown, bool(o.overflow), bool(o.needs_resort), o.tail_start))
    return static, o, flags, overflows


@pytest.mark.parametrize("name", sorted(cc.CONFIGS))
def test_oracle_reproduces_the_pinned_claim_digest(oracle, name: str) -> None:
    _, o, _, overflows = _oracle_run(oracle, name)
    assert cc.digest(o.conns, o.needs_resort, overflows) == cc.GOLDEN[name]


def test_the_configs_exercise_overflow_and_resort(oracle) -> None:
    """test_growth_claim.py:330-344."""
    _, _, _, overflows = _oracle_run(oracle, "propose_overflow")
    assert any(overflows) and not all(overflows)
    _, static, _ = cc.build("propose_small_claim", "cpu")
    k = cc.CONFIGS["propose_small_claim"]["k"]
    assert all(k * 1024 <= cap for cap in static.level_capacities[:-1])
    _, static, _ = cc.build("propose_window2", "cpu")
    assert any(cap % 64 for cap in static.level_capacities)
    _, o, _, _ = _oracle_run(oracle, "propose_window2")
    assert o.needs_resort


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(cc.CONFIGS))
def test_device_reproduces_the_pinned_claim_digest(oracle, name: str) -> None:
    import plastax_amd as px

    _, _, want_flags, _ = _oracle_run(oracle, name)
    net, static, state = cc.build(name, "cuda")
    step = px.make_step(net, static)
    x = np.ones(len(static.input_ids), np.float32)
    overflows = []
    print(f"claim digest {name}", flush=True)
    for k in range(cc.STEPS):
        state = step(state, px.StepInputs(x, None)).state
        overflows.append(bool(state.overflow))
        got = (state.grown, bool(state.overflow), bool(state.needs_resort), state.tail_start)
        assert got == want_flags[k], f"flags at step {k + 1}"
    assert cc.digest(state.conns, state.needs_resort, overflows) == cc.GOLDEN[name]
