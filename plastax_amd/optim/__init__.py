"""Optimizer bundles (src/plastax/optim/__init__.py:1-77).

Each bundle is an ``UpdateConn`` policy plus the per-connection state
columns it needs (``state_fields``, merged into a Network's
``extra_conn_fields``). The device runs them as fused per-edge update rules
(PLX_RULE_* in include/plastax_hip.h); the float32 operation order of each
rule is the reference's (cited on each ``_step``).
"""

from __future__ import annotations

from plastax_amd.optim._rules import (
    SGD,
    Adam,
    Momentum,
    Optimizer,
    RMSProp,
    adam,
    adamw,
    momentum,
    rmsprop,
    sgd,
)

__all__ = [
    "SGD",
    "Adam",
    "Momentum",
    "Optimizer",
    "RMSProp",
    "adam",
    "adamw",
    "momentum",
    "rmsprop",
    "sgd",
]
