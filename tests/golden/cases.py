"""Golden cases: one attention layer of each BASELINE model family, end to end.

Each case draws its inputs from the seeded generator (spissa_amd.synth), runs
the reference pipeline of one layer on the CPU oracle and records the result in
fixtures.json (written by make_fixtures.py):

  llama  (models/llama/generate.rs:383-416): RoPE of the cached keys at their
         positions and of q/k at position P.. (rotary.rs:75-125), attention
         over cache + current rows (rotary.rs:335-415), append (rotary.rs:226-256).
  gemma  (models/gemma/generate.rs:232-295): per-head RMSNorm of q and k
         (ops.rs:159-179), Gemma RoPE with the layer's base and position
         divisor (rotary.rs:137-186), q prescale (x1.0 for
         query_pre_attn_scalar == head_dim), attention with the layer's sliding
         window (0 on global layers), append.

Past keys are drawn before RoPE and rotated at their absolute positions, as a
real cache would hold them. QK-norm weights are effective multipliers drawn
from N(1, 0.1).
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np

from spissa_amd.synth import normal_f32, seed_for

EPS = 1e-6


@dataclass(frozen=True)
class Case:
    name: str
    config: int      # BASELINE config index (1-based) the geometry comes from
    kind: str        # "llama" or "gemma"
    Hq: int
    Hkv: int
    D: int
    P: int           # cached tokens before the call
    S: int           # tokens in the call
    base: float
    divisor: float = 1.0
    window: int = 0
    layer: int = 0

    @property
    def n_out(self) -> int:
        return self.S * self.Hq * self.D


CASES = [
    Case("llama1b_decode_p512", 1, "llama", 32, 8, 64, 512, 1, 500000.0),
    Case("llama3b_decode_p8192", 3, "llama", 24, 8, 128, 8192, 1, 500000.0),
    Case("llama1b_prefill_s256", 2, "llama", 32, 8, 64, 0, 256, 500000.0),
    Case("llama3b_chunk_s64_p300", 3, "llama", 24, 8, 128, 300, 64, 500000.0),
    Case("gemma1b_local_decode_p2048_w512", 4, "gemma", 4, 1, 256, 2048, 1, 10000.0, 1.0, 512, 0),
    Case("gemma1b_global_decode_p4096", 4, "gemma", 4, 1, 256, 4096, 1, 1000000.0, 8.0, 0, 5),
    Case("gemma4b_chunk_s16_p1024_w1024", 5, "gemma", 8, 4, 256, 1024, 16, 10000.0, 1.0, 1024, 0),
]


def raw_inputs(c: Case):
    """Pre-RoPE draws: q [S,Hq,D], k/v [P+S,Hkv,D] (past rows first), norm weights [D]."""
    q = normal_f32(seed_for(c.config, c.layer, 0, "q"), c.S * c.Hq * c.D)
    k = normal_f32(seed_for(c.config, c.layer, 0, "k"), (c.P + c.S) * c.Hkv * c.D)
    v = normal_f32(seed_for(c.config, c.layer, 0, "v"), (c.P + c.S) * c.Hkv * c.D)
    qn = normal_f32(seed_for(c.config, c.layer, 0, "qnorm"), c.D, 1.0, 0.1)
    kn = normal_f32(seed_for(c.config, c.layer, 0, "knorm"), c.D, 1.0, 0.1)
    return q, k, v, qn, kn


def sha(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a, dtype=np.float32).tobytes())
    return h.hexdigest()


def sample_index(n: int, count: int = 512) -> np.ndarray:
    """Fixed sample positions of an output of n elements (all of them when small)."""
    if n <= count:
        return np.arange(n)
    return np.unique(np.linspace(0, n - 1, count).astype(np.int64))


def run_oracle(c: Case, o):
    """The layer on the CPU oracle `o`: returns (out, cache keys, cache values)."""
    q, k, v, qn, kn = raw_inputs(c)
    w = c.Hkv * c.D
    kp, kc = k[:c.P * w].copy(), k[c.P * w:].copy()
    vp, vc = v[:c.P * w].copy(), v[c.P * w:].copy()
    if c.kind == "llama":
        if c.P:
            dummy = np.zeros(c.P * c.D, dtype=np.float32)  # RoPE of the past keys alone
            o.apply_llama_rotary_inplace(kp, dummy, c.Hkv, 1, c.P, c.D, c.D, c.base, 0)
        o.apply_llama_rotary_inplace(q, kc, c.Hq, c.Hkv, c.S, c.D, c.D, c.base, c.P)
    else:
        if c.P:
            dummy = np.zeros(c.P * c.D, dtype=np.float32)
            o.gemma_qk_prologue(dummy, kp, c.P, 1, c.Hkv, c.D, qn, kn, EPS, c.base, c.divisor, 0, float(c.D))
        o.gemma_qk_prologue(q, kc, c.S, c.Hq, c.Hkv, c.D, qn, kn, EPS, c.base, c.divisor, c.P, float(c.D))
    cache = o.KvCache(c.Hkv, c.D, c.P + c.S)
    if c.P:
        cache.append(kp, vp, c.P)
    out = o.sdpa_with_cache(q, kc, vc, cache, c.S, c.Hq, c.Hkv, c.D, True, c.window)
    cache.append(kc, vc, c.S)
    return out, cache.keys(), cache.values()
