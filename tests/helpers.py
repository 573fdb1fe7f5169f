"""Shared helpers for the parity tests."""
from __future__ import annotations

import numpy as np

from spissa_amd.synth import normal_f32, seed_for


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max|got - ref| / max|ref| over the whole tensor (the tolerance metric)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = np.max(np.abs(ref))
    if denom == 0:
        return float(np.max(np.abs(got - ref)))
    return float(np.max(np.abs(got - ref)) / denom)


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bitwise(got: np.ndarray, ref: np.ndarray, what: str = "") -> None:
    g, r = bits(got), bits(ref)
    assert g.shape == r.shape, f"{what}: shape {g.shape} != {r.shape}"
    bad = np.nonzero(g != r)[0]
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} elements differ; first at {bad[0]}: "
                           f"{got.ravel()[bad[0]]!r} vs {ref.ravel()[bad[0]]!r}")


def layer_inputs(config: int, layer: int, S: int, P: int, Hq: int, Hkv: int, D: int, turn: int = 0,
                 sequence: int = 0):
    """Seeded q [S,Hq,D], cur k/v [S,Hkv,D] and past k/v [P,Hkv,D], all N(0,1) float32."""
    q = normal_f32(seed_for(config, layer, turn, "q", sequence), S * Hq * D)
    kv_k = normal_f32(seed_for(config, layer, turn, "k", sequence), (P + S) * Hkv * D)
    kv_v = normal_f32(seed_for(config, layer, turn, "v", sequence), (P + S) * Hkv * D)
    w = Hkv * D
    return q, kv_k[P * w:].copy(), kv_v[P * w:].copy(), kv_k[:P * w].copy(), kv_v[:P * w].copy()
