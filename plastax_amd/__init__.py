"""plastax_amd: the MI355X-native streaming edge-arena step of plastax.

The public names mirror the reference's API (src/plastax/__init__.py:52-105)
for the path this package implements: declare a ``Network`` subclass, build
it with ``NetworkBuilder.from_edges``, and run ``make_step(net, static)``.
The step's edge work runs in hand-written gfx950 HIP kernels
(libplastax_hip.so, C ABI in include/plastax_hip.h); there is no CPU
fallback.
"""

from __future__ import annotations

from plastax_amd import monoid, nn, numpy, optim, rng, topo
from plastax_amd._expr import UnsupportedPolicyError
from plastax_amd._types import (
    ACTIVATION,
    DEAD,
    FROM_ID,
    LEVEL,
    PRUNED,
    TO_ID,
    WEIGHT,
    ConnIdx,
    FieldSpec,
    Level,
    Propagation,
    ShardSpec,
    UnitIdx,
)
from plastax_amd.builder import NetworkBuilder
from plastax_amd.driver import Driver
from plastax_amd.growth_config import (
    ShortlistCoverage,
    predicate_add_conn,
    recommended_shortlist,
    shortlist_coverage,
)
from plastax_amd.monoid import Monoid, UnsupportedMonoidError
from plastax_amd.state import (
    NetworkState,
    NetworkStatic,
    grow_bucket,
    live_conn_count,
    live_unit_count,
    live_unit_mask,
    make_empty_state,
)
from plastax_amd.step import StepInputs, StepResult, make_step
from plastax_amd.traits import (
    AddUnit,
    BackwardPass,
    BatchReduction,
    FieldReductions,
    ForwardPass,
    Loss,
    MeanFloatFirstRest,
    Network,
    Proposal,
    ProposeAddConn,
    PruneConn,
    PruneUnit,
    Reduction,
    ResetGlobal,
    ScoreAddConn,
    SoftmaxCrossEntropyLoss,
    UpdateConn,
    UpdateUnit,
)
from plastax_amd.views import ConnView, ConnWrite, UnitView, UnitWrite

__all__ = [
    "ACTIVATION",
    "DEAD",
    "FROM_ID",
    "LEVEL",
    "PRUNED",
    "TO_ID",
    "WEIGHT",
    "AddUnit",
    "BackwardPass",
    "BatchReduction",
    "FieldReductions",
    "Reduction",
    "Driver",
    "ConnIdx",
    "ConnView",
    "ConnWrite",
    "FieldSpec",
    "ForwardPass",
    "Level",
    "Loss",
    "MeanFloatFirstRest",
    "Monoid",
    "Network",
    "NetworkBuilder",
    "NetworkState",
    "NetworkStatic",
    "Propagation",
    "Proposal",
    "ProposeAddConn",
    "PruneConn",
    "PruneUnit",
    "ResetGlobal",
    "ScoreAddConn",
    "ShardSpec",
    "ShortlistCoverage",
    "SoftmaxCrossEntropyLoss",
    "StepInputs",
    "StepResult",
    "UnitIdx",
    "UnitView",
    "UnitWrite",
    "UnsupportedMonoidError",
    "UnsupportedPolicyError",
    "UpdateConn",
    "UpdateUnit",
    "grow_bucket",
    "live_conn_count",
    "live_unit_count",
    "live_unit_mask",
    "make_empty_state",
    "make_step",
    "monoid",
    "nn",
    "numpy",
    "optim",
    "predicate_add_conn",
    "recommended_shortlist",
    "rng",
    "shortlist_coverage",
    "topo",
]
