"""Synthetic workloads of the benchmark configurations.

``c1_pipeline`` and ``c2_topological`` build the edge lists of the first two
configurations with numpy's PCG64 (seed 0 by default), so the same arrays are
reproducible on any host:

- C1: 1,024 units; 16,384 edges with uniform src/dst and no self-loops;
  PIPELINE tanh; 32 inputs, 8 outputs; weights N(0, 1/fan_in).
- C3: the batched sparse MLP 784-4096-4096-10 with each layer pair's
  dense edges kept with probability 0.1 (about 2.0M edges), weights
  N(0, 1/fan_in); inputs uniform in [0, 1); labels the argmax of a fixed
  random linear teacher of the inputs.
- C2: 8 layers x 131,072 units (layer 0 = inputs, layer 7 = outputs);
  2^26 edges between consecutive layers, fan-in 73 plus one more for every
  7th destination; each destination's sources are drawn without replacement
  by Zipf(s=1.1) popularity over a seeded permutation of the source layer;
  weights N(0, 1/fan_in).

``scale`` shrinks the layer width (and with it the edge count) for tests.
"""

from __future__ import annotations

import dataclasses

import numpy as np


@dataclasses.dataclass
class EdgeList:
    num_units: int
    src: np.ndarray  # int32
    dst: np.ndarray  # int32
    weight: np.ndarray  # float32
    input_ids: np.ndarray
    output_ids: np.ndarray


def c1_pipeline(seed: int = 0, num_units: int = 1024, num_edges: int = 16384,
                n_in: int = 32, n_out: int = 8) -> EdgeList:
    """C1's recurrent pipeline net."""
    rng = np.random.default_rng(seed)
    src = rng.integers(0, num_units, size=num_edges, dtype=np.int64)
    dst = rng.integers(0, num_units - 1, size=num_edges, dtype=np.int64)
    dst = dst + (dst >= src)  # uniform over the other units: no self-loops
    fan_in = np.bincount(dst, minlength=num_units)
    std = 1.0 / np.sqrt(np.maximum(fan_in[dst], 1))
    weight = (rng.standard_normal(num_edges) * std).astype(np.float32)
    return EdgeList(
        num_units,
        src.astype(np.int32),
        dst.astype(np.int32),
        weight,
        np.arange(n_in, dtype=np.int32),
        np.arange(num_units - n_out, num_units, dtype=np.int32),
    )


def zipf_sources(rng: np.random.Generator, width: int, counts: np.ndarray,
                 s: float = 1.1, oversample: int = 160) -> tuple[np.ndarray, np.ndarray]:
    """For destination row r, ``counts[r]`` distinct source ranks drawn
    sequentially by Zipf(s) popularity (rank k has weight k^-s), mapped
    through a random permutation of the layer. Returns (row, source) pairs."""
    cdf = np.cumsum(np.arange(1, width + 1, dtype=np.float64) ** -s)
    cdf /= cdf[-1]
    perm = rng.permutation(width).astype(np.int32)
    rows_out, src_out = [], []
    n = counts.size
    need = counts.astype(np.int64)
    if int(need.max(initial=0)) > width:
        raise ValueError("more distinct sources requested than the layer holds")
    pending = np.arange(n)
    chunk = 4096
    rounds = 0
    while pending.size:
        next_pending = []
        # rows that found too few distinct sources retry with twice the draws
        k_round = int(max(oversample, 2 * need.max(initial=0))) << rounds
        rounds += 1
        for c0 in range(0, pending.size, max(1, chunk >> (rounds - 1))):
            rows = pending[c0 : c0 + max(1, chunk >> (rounds - 1))]
            k = k_round
            u = rng.random((rows.size, k))
            draws = np.searchsorted(cdf, u, side="right").astype(np.int32)
            np.minimum(draws, width - 1, out=draws)
            order = np.argsort(draws, axis=1, kind="stable")
            srt = np.take_along_axis(draws, order, axis=1)
            dup_sorted = np.zeros_like(srt, dtype=bool)
            dup_sorted[:, 1:] = srt[:, 1:] == srt[:, :-1]
            dup = np.zeros_like(dup_sorted)
            np.put_along_axis(dup, order, dup_sorted, axis=1)
            keep = ~dup
            rank = np.cumsum(keep, axis=1)
            take = keep & (rank <= need[rows][:, None])
            ok = take.sum(axis=1) == need[rows]
            r_idx, c_idx = np.nonzero(take & ok[:, None])
            rows_out.append(rows[r_idx])
            src_out.append(perm[draws[r_idx, c_idx]])
            next_pending.append(rows[~ok])
        pending = np.concatenate(next_pending) if next_pending else np.zeros(0, np.int64)
    return np.concatenate(rows_out), np.concatenate(src_out)


def c2_topological(seed: int = 0, scale: int = 1, layers: int = 8) -> EdgeList:
    """C2's 8-layer Zipf net (2^26 edges at scale 1)."""
    rng = np.random.default_rng(seed)
    width = 131072 // scale
    num_units = layers * width
    src_all, dst_all, w_all = [], [], []
    for layer in range(layers - 1):
        counts = np.full(width, 73, dtype=np.int64)
        # every 7th of the (layers-1)*width destinations gets one more source
        counts[((layer * width + np.arange(width)) % 7) == 0] += 1
        rows, srcs = zipf_sources(rng, width, counts)
        dst = (layer + 1) * width + rows.astype(np.int64)
        src = layer * width + srcs.astype(np.int64)
        std = 1.0 / np.sqrt(counts[rows].astype(np.float64))
        w = (rng.standard_normal(rows.size) * std).astype(np.float32)
        src_all.append(src.astype(np.int32))
        dst_all.append(dst.astype(np.int32))
        w_all.append(w)
    return EdgeList(
        num_units,
        np.concatenate(src_all),
        np.concatenate(dst_all),
        np.concatenate(w_all),
        np.arange(width, dtype=np.int32),
        np.arange((layers - 1) * width, layers * width, dtype=np.int32),
    )


def c3_mlp(seed: int = 0, layers: tuple[int, ...] = (784, 4096, 4096, 10), keep: float = 0.1) -> EdgeList:
    """C3's sparse MLP (each dense layer pair's edge kept w.p. ``keep``)."""
    rng = np.random.default_rng(seed)
    base = np.concatenate([[0], np.cumsum(layers)])
    src_all, dst_all = [], []
    for l in range(len(layers) - 1):
        m = rng.random((layers[l], layers[l + 1])) < keep
        ii, jj = np.nonzero(m)
        src_all.append((base[l] + ii).astype(np.int32))
        dst_all.append((base[l + 1] + jj).astype(np.int32))
    src = np.concatenate(src_all)
    dst = np.concatenate(dst_all)
    fan = np.bincount(dst, minlength=int(base[-1]))
    w = (rng.standard_normal(src.size) / np.sqrt(np.maximum(fan[dst], 1))).astype(np.float32)
    return EdgeList(int(base[-1]), src, dst, w, np.arange(layers[0], dtype=np.int32),
                    np.arange(base[-2], base[-1], dtype=np.int32))


def c3_batches(seed: int, steps: int, batch: int, n_in: int = 784, n_out: int = 10):
    """C3's synthetic batches: inputs uniform in [0, 1), one-hot labels of a
    fixed random linear teacher's argmax."""
    rng = np.random.default_rng(seed + 1)
    teacher = rng.standard_normal((n_out, n_in)).astype(np.float32)
    xs = rng.random((steps, batch, n_in)).astype(np.float32)
    lab = np.argmax(xs @ teacher.T, axis=-1)
    ys = np.eye(n_out, dtype=np.float32)[lab]
    return xs, ys


def c2_target(seed: int, width: int):
    """The fixed linear target of C2: y_k = s_k * x_{pi(k)}."""
    rng = np.random.default_rng(seed + 1)
    sign = np.where(rng.random(width) < 0.5, -1.0, 1.0).astype(np.float32)
    perm = rng.permutation(width)
    return sign, perm


def c1_target(seed: int, n_in: int = 32, n_out: int = 8) -> np.ndarray:
    """C1's fixed random linear target matrix A (n_out x n_in), N(0, 1/n_in)."""
    rng = np.random.default_rng(seed + 1)
    return (rng.standard_normal((n_out, n_in)) / np.sqrt(n_in)).astype(np.float32)


def c5_reservoir(seed: int = 0, num_units: int = 65536, num_edges: int = 4 * 1024 * 1024,
                 n_in: int = 256) -> EdgeList:
    """C5's growing reservoir at its starting shape: 65,536 live units, 4M
    uniform random recurrent edges without self-loops (PIPELINE), weights
    N(0, 1) scaled by 1/sqrt(mean fan-in) so the spectral radius is about 1;
    256 inputs. The unit and edge capacities (262,144 and 16M) are the
    builder's (unit_capacity, capacity_headroom=3)."""
    rng = np.random.default_rng(seed)
    src = rng.integers(0, num_units, size=num_edges, dtype=np.int64)
    dst = rng.integers(0, num_units - 1, size=num_edges, dtype=np.int64)
    dst = dst + (dst >= src)
    scale = 1.0 / np.sqrt(num_edges / num_units)
    weight = (rng.standard_normal(num_edges) * scale).astype(np.float32)
    return EdgeList(
        num_units,
        src.astype(np.int32),
        dst.astype(np.int32),
        weight,
        np.arange(n_in, dtype=np.int32),
        np.arange(num_units - 16, num_units, dtype=np.int32),
    )
