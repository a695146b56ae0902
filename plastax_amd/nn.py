"""jax.nn-style activations for device-traceable policies."""

from __future__ import annotations

from typing import Any

import numpy as np

from plastax_amd._expr import Expr, unary


def sigmoid(x: Any) -> Any:
    """1 / (1 + exp(-x)), as jax.nn.sigmoid (lax.logistic)."""
    if isinstance(x, Expr):
        return unary("sigmoid", x)
    x = np.float32(x)
    return np.float32(1.0) / (np.float32(1.0) + np.exp(-x))


def relu(x: Any) -> Any:
    """max(x, 0), as jax.nn.relu."""
    if isinstance(x, Expr):
        return unary("relu", x)
    return np.maximum(np.float32(x), np.float32(0.0))


def tanh(x: Any) -> Any:
    if isinstance(x, Expr):
        return unary("tanh", x)
    return np.tanh(np.float32(x))
