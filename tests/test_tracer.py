"""The policy tracer: what compiles to a device program and what is refused
(the reference's trace-time contracts: linear_input, phases.py:535-556;
named monoids only, monoid.py:206-218)."""

from __future__ import annotations

import numpy as np
import pytest

import nets
import plastax_amd as px
import plastax_amd.numpy as jnp
from plastax_amd._expr import OPCODES, Index, UnsupportedPolicyError
from plastax_amd._plan import compile_plan


def _ops(prog) -> list[str]:
    names = {v: k for k, v in OPCODES.items()}
    return [names[c[0]] for c in prog.code]


def _static(net):
    static, _ = px.NetworkBuilder.from_edges(
        net, 3, np.int32([0, 1]), np.int32([2, 2]), weights=np.float32([1, 1]),
        input_ids=[0, 1], output_ids=[2], globals_=None, device="cpu")
    return static


def test_relu_net_plan() -> None:
    plan = compile_plan(nets.ReluMlpNet, _static(nets.ReluMlpNet))
    assert plan.forward.field == "activation" and plan.forward.monoid == 0
    assert plan.backward.field == "grad_pre_act"
    assert _ops(plan.forward.program) == ["acc", "const", "max", "out"]
    assert plan.forward.program.out_fields == ["activation"]
    # (acc + loss_grad) * where(act > 0, 1, 0)
    ops = _ops(plan.backward.program)
    assert ops.count("sel") == 1 and "gt" in ops and ops[-1] == "out"
    assert set(plan.backward.program.fields) == {"activation", "loss_grad"}
    # MSE: seed = pred - target; term = 0.5 * diff * diff
    lp = plan.loss
    assert lp.kind == "elementwise" and lp.seed_field == "loss_grad"
    assert _ops(lp.program) == ["ldu", "target", "sub", "const", "mul", "mul", "out", "out"]


def test_softmax_loss_is_its_own_kernel() -> None:
    plan = compile_plan(nets.SoftmaxNet, _static(nets.SoftmaxNet))
    assert plan.loss.kind == "softmax" and plan.loss.program is None


def test_nonlinear_map_runs_as_a_generic_pass() -> None:
    class SquareMap(px.ForwardPass):
        def map(self, u, dst, src, c, cid, g):
            return c[px.WEIGHT, cid] * u[px.ACTIVATION, src] * u[px.ACTIVATION, src]

        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((px.ACTIVATION, acc))

    class Net(px.Network):
        forward_pass = SquareMap()

    plan = compile_plan(Net, _static(Net))
    assert plan.forward.generic is not None and "map must be" in plan.forward.generic.why


def test_generic_monoid_is_refused() -> None:
    class Gen(nets.LinearForward):
        combine = px.Monoid(None, op=lambda a, b: a + b, identity=0.0)

    class Net(px.Network):
        forward_pass = Gen()

    with pytest.raises(px.UnsupportedMonoidError):
        compile_plan(Net, _static(Net))


def test_python_control_flow_on_traced_values_is_refused() -> None:
    class Branchy(nets.LinearForward):
        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((px.ACTIVATION, acc if acc > 0 else -acc))

    class Net(px.Network):
        forward_pass = Branchy()

    with pytest.raises(UnsupportedPolicyError):
        compile_plan(Net, _static(Net))


def test_reading_another_units_field_in_apply_is_refused() -> None:
    class Peek(nets.LinearForward):
        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((px.ACTIVATION, acc + u[px.ACTIVATION, Index("src")]))

    class Net(px.Network):
        forward_pass = Peek()

    with pytest.raises(UnsupportedPolicyError):
        compile_plan(Net, _static(Net))


def test_globals_become_refreshed_constants() -> None:
    class Scaled(nets.LinearForward):
        def apply(self, u, i, g, acc):
            return px.UnitWrite.of((px.ACTIVATION, jnp.tanh(acc * g["gain"])))

    class Net(px.Network):
        forward_pass = Scaled()

    prog = compile_plan(Net, _static(Net)).forward.program
    assert list(prog.globals_at.values()) == ["gain"]
    slot = next(iter(prog.globals_at))
    assert prog.const_values({"gain": 2.5})[slot] == np.float32(2.5)
    assert prog.const_values({"gain": -1.0})[slot] == np.float32(-1.0)


def test_unsupported_phases_fail_at_build() -> None:
    class Pr(px.PruneConn):
        def predicate(self, u, c, cid, g):
            return abs(c[px.WEIGHT, cid]) < 0.1

    class Net(nets.ReluMlpNet):
        update_unit = object()

    with pytest.raises(TypeError):
        compile_plan(Net, _static(Net))

    class Net2(nets.ReluMlpNet):
        prune_conn = Pr()
        update_conn = nets.px.optim.sgd(1e-2, nets.GRAD_PRE_ACT).update_conn()

    plan = compile_plan(Net2, _static(Net2))
    assert plan.prune_conn and not plan.update_unit

    class Normal(px.ProposeAddConn):
        proposals_per_proposer = 1
        max_new_per_level = 1

        def propose(self, u, i, j, g, rng):
            return i, i, rng.normal()

        def init(self, u, src, dst, g):
            return px.ConnWrite.of()

    from plastax_amd import _site

    # Rng.normal is Box-Muller on two draws (rng.py:289-299): two rng reads,
    # then log, sqrt and cos, in the reference's float32 op order.
    prog = _site.trace_propose(Normal(), "per_unit", {"activation": np.dtype(np.float32)}, {}, None)
    ops = [c[0] for c in prog.code]
    assert ops.count(_site.SOP["rng"]) == 2
    for name in ("flog", "fsqrt", "fcos"):
        assert _site.SOP[name] in ops


def test_register_reuse_keeps_long_programs_in_budget() -> None:
    class Long(nets.LinearForward):
        def apply(self, u, i, g, acc):
            v = acc
            for k in range(9):
                v = jnp.tanh(v * np.float32(1.0 + k / 16)) + acc
            return px.UnitWrite.of((px.ACTIVATION, v))

    class Net(px.Network):
        forward_pass = Long()

    prog = compile_plan(Net, _static(Net)).forward.program
    assert max(max(c[1], c[2], c[3]) for c in prog.code) < 16
