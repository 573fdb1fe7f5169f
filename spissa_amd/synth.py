"""Seeded synthetic inputs: splitmix64 -> Box-Muller -> float32 N(mean, std).

The same seed gives the same bytes on every host, so the CPU oracle and the
GPU path are fed identical Q/K/V. Seeds are derived from
(config, layer, turn, tensor, sequence).
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
TENSORS = {"q": 1, "k": 2, "v": 3, "qnorm": 4, "knorm": 5}


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """The n outputs of a splitmix64 stream seeded with `seed`, starting at `offset`."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        return _mix(np.uint64(seed) + i * _GOLDEN)


def seed_for(config: int, layer: int = 0, turn: int = 0, tensor: str = "q", sequence: int = 0) -> int:
    """Deterministic 64-bit seed of one tensor of one (config, layer, turn, sequence)."""
    with np.errstate(over="ignore"):
        s = np.uint64(0x5350495353410000)  # "SPISSA"
        for part in (config, layer, turn, TENSORS[tensor], sequence):
            s = _mix(np.array([s ^ np.uint64(part & 0xFFFFFFFFFFFFFFFF)], dtype=np.uint64))[0]
    return int(s)


def normal_f32(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """n float32 draws of N(mean, std^2) (Box-Muller on f64, rounded once)."""
    a = splitmix64(seed, n)
    b = splitmix64(seed, n, offset=n)
    u1 = ((a >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u2 = (b >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (mean + std * z).astype(np.float32)
