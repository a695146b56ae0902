"""Counter-based Philox-4x32-10 draws (src/plastax/rng.py:1-309).

The site-keying contract (rng.py:10-56): a draw is
``philox32(site_seed, (j << 16) | sub)`` with
``site_seed = (philox32(net_seed, (step << 8) | stream) << 32) | key``.
Host-side words are computed vectorised in numpy (uint64 arithmetic); the
device computes the same words (``plx_philox32``).
"""

from __future__ import annotations

import numpy as np

_M0 = np.uint64(0xD2511F53)
_M1 = np.uint64(0xCD9E8D57)
_W0 = np.uint32(0x9E3779B9)
_W1 = np.uint32(0xBB67AE85)
_MASK = np.uint64(0xFFFFFFFF)


def philox32(seed: np.ndarray | int, counter: np.ndarray | int) -> np.ndarray:
    """First word of Philox-4x32-10 with the counter block
    (ctr_lo, ctr_hi, seed_lo, seed_hi) and key (seed_lo, seed_hi)
    (rng.py:109-141). Vectorised over numpy uint64 inputs."""
    seed = np.asarray(seed, dtype=np.uint64)
    counter = np.asarray(counter, dtype=np.uint64)
    seed, counter = np.broadcast_arrays(seed, counter)
    x0 = (counter & _MASK).astype(np.uint32)
    x1 = (counter >> np.uint64(32)).astype(np.uint32)
    x2 = (seed & _MASK).astype(np.uint32)
    x3 = (seed >> np.uint64(32)).astype(np.uint32)
    k0 = x2.copy()
    k1 = x3.copy()
    with np.errstate(over="ignore"):
        for _ in range(10):
            p0 = _M0 * x0.astype(np.uint64)
            p1 = _M1 * x2.astype(np.uint64)
            hi0 = (p0 >> np.uint64(32)).astype(np.uint32)
            lo0 = (p0 & _MASK).astype(np.uint32)
            hi1 = (p1 >> np.uint64(32)).astype(np.uint32)
            lo1 = (p1 & _MASK).astype(np.uint32)
            x0, x1, x2, x3 = hi1 ^ x1 ^ k0, lo1, hi0 ^ x3 ^ k1, lo0
            k0 = k0 + _W0
            k1 = k1 + _W1
    return x0


def unit_float(word: np.ndarray) -> np.ndarray:
    """float32(word >> 8) * 2^-24 in [0, 1) (rng.py:144-153)."""
    w = np.asarray(word, dtype=np.uint32)
    return (w >> np.uint32(8)).astype(np.float32) * np.float32(1.0 / 16777216.0)


def conn_key(src: np.ndarray, dst: np.ndarray, occurrence: np.ndarray) -> np.ndarray:
    """philox32((src << 32) | dst, occurrence) (rng.py:156-180)."""
    s = np.asarray(src).astype(np.uint64)
    d = np.asarray(dst).astype(np.uint64) & _MASK
    return philox32((s << np.uint64(32)) | d, np.asarray(occurrence).astype(np.uint64))


def site_seed(network_seed: int, step: np.ndarray | int, stream: int, key: np.ndarray) -> np.ndarray:
    """(philox32(net_seed, (step << 8) | stream) << 32) | key (rng.py:206-246)."""
    ctr = (np.asarray(step).astype(np.uint64) << np.uint64(8)) | np.uint64(stream & 0xFF)
    hi = philox32(np.uint64(network_seed & 0xFFFFFFFFFFFFFFFF), ctr).astype(np.uint64)
    return (hi << np.uint64(32)) | (np.asarray(key).astype(np.uint64) & _MASK)


def draw(site: np.ndarray, j: np.ndarray, sub: int) -> np.ndarray:
    """philox32(site, (j << 16) | sub) (rng.py:248-259)."""
    ctr = (np.asarray(j).astype(np.uint64) << np.uint64(16)) | np.uint64(sub & 0xFFFF)
    return philox32(site, ctr)


def uniform_int(word: np.ndarray, n: int) -> np.ndarray:
    """min(uint32(u * n), n - 1) (rng.py:273-287)."""
    scaled = (unit_float(word) * np.float32(n)).astype(np.uint32)
    return np.minimum(scaled, np.uint32(n - 1))
