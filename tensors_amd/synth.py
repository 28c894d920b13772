"""Seeded synthetic inputs for the benchmark configurations.

A counter-based generator (SplitMix64 of seed + counter) with explicit
transforms, so the same tensor is produced on any host and by any consumer:

* ``uint64(seed, n)``    — z_i = splitmix64(seed + (i+1) * golden)
* ``uniform_int``        — floor(hi32(z) * n / 2^32)  (multiply-high)
* ``normal``             — Box-Muller in float64 from two draws, rounded to f32
* ``mnist_like``         — (U{0..255} * (1/255) - 0.1307) * (1/0.3081), each
  constant and operation in float32 as in
  data/MnistLoader.cpp:73-80 of the reference.

Seeds follow ``seed(config, tensor_id) = 0x7E450000 + 16 * config + tensor_id``.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def seed(config: int, tensor_id: int) -> int:
    return 0x7E450000 + 16 * config + tensor_id


def uint64(seed_: int, n: int, offset: int = 0) -> np.ndarray:
    i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed_) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform_int(seed_: int, shape, n: int, offset: int = 0) -> np.ndarray:
    count = int(np.prod(shape))
    hi = uint64(seed_, count, offset) >> np.uint64(32)
    return ((hi * np.uint64(n)) >> np.uint64(32)).astype(np.int64).reshape(shape)


def normal(seed_: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    count = int(np.prod(shape))
    z = uint64(seed_, 2 * count)
    u1 = ((z[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)
    u2 = (z[1::2] >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
    n = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (mean + std * n).astype(np.float32).reshape(shape)


def mnist_like(seed_: int, shape) -> np.ndarray:
    inv255 = np.float32(1.0) / np.float32(255.0)
    inv_std = np.float32(1.0) / np.float32(0.3081)
    px = uniform_int(seed_, shape, 256).astype(np.float32) * inv255
    return (px - np.float32(0.1307)) * inv_std
