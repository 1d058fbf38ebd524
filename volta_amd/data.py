"""Seeded synthetic inputs and weights for the benchmark configurations.

Generators (all deterministic across machines, numpy uint64 arithmetic):
  * splitmix64 stream -> U(0,1) from the top 53 bits / 2**53;
  * N(0,1) by Box-Muller in float64, cast to float32;
  * He-uniform weights U(-sqrt(6/fan_in), +sqrt(6/fan_in)), zero biases;
  * class labels as u64 % C.

The reference's own initialiser (LCG Xavier-uniform, seed 42,
mlp_train_rust_codegen.rs:629-658) is what volta_train_init applies; the
benchmark configurations ask for He-uniform instead, which callers inject
through volta_train_set_params.
"""
from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, count: int) -> np.ndarray:
    """`count` outputs of splitmix64 started from `seed`."""
    with np.errstate(over="ignore"):
        idx = np.arange(1, count + 1, dtype=np.uint64)
        z = np.uint64(seed) + idx * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform01(seed: int, count: int) -> np.ndarray:
    """float64 in [0, 1)."""
    return (splitmix64(seed, count) >> np.uint64(11)).astype(np.float64) / float(1 << 53)


def normal(seed: int, shape) -> np.ndarray:
    """float32 N(0,1) by Box-Muller."""
    count = int(np.prod(shape))
    pairs = (count + 1) // 2
    u = uniform01(seed, 2 * pairs)
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    rad = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * pairs, dtype=np.float64)
    z[0::2] = rad * np.cos(2.0 * np.pi * u2)
    z[1::2] = rad * np.sin(2.0 * np.pi * u2)
    return z[:count].astype(np.float32).reshape(shape)


def labels(seed: int, batch: int, classes: int) -> np.ndarray:
    return (splitmix64(seed, batch) % np.uint64(classes)).astype(np.int32)


def he_uniform(seed: int, sizes: Sequence[int]) -> Tuple[List[np.ndarray], List[np.ndarray]]:
    """He-uniform W_i [r x c] per layer (fan_in = r), zero biases."""
    ws, bs = [], []
    for i in range(len(sizes) - 1):
        r, c = int(sizes[i]), int(sizes[i + 1])
        lim = np.sqrt(6.0 / r)
        u = uniform01(seed * 1000003 + 17 * (i + 1), r * c)
        ws.append(((2.0 * u - 1.0) * lim).astype(np.float32).reshape(r, c))
        bs.append(np.zeros(c, dtype=np.float32))
    return ws, bs


def batch(seed: int, sizes: Sequence[int], batch_size: int, loss: str):
    """(X [B x L0], Y) with Y ~ N(0,1) [B x Ln] for MSE or int32 labels for CE."""
    X = normal(seed * 7919 + 1, (batch_size, int(sizes[0])))
    if loss == "ce":
        Y = labels(seed * 7919 + 2, batch_size, int(sizes[-1]))
    else:
        Y = normal(seed * 7919 + 2, (batch_size, int(sizes[-1])))
    return X, Y
