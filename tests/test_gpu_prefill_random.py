"""Seeded random prefill shapes against the CPU oracle.

The launch plan picks the kernel shape per call: wave pairs, key splits and
their count, the XCD grouping, the head_dim-256 stage count. This sweeps
shapes across those choices (head dims 64/128/256, GQA ratios 1-8, prompts
and chunks over caches, causal or not, with and without a window) so that
every combination the plan can produce meets the bf16 bar:
max|gpu - ref| / max|ref| <= 1e-2 (the same metric as test_gpu_attention.py).
"""
import numpy as np
import pytest

import oracle as o
from tests.helpers import layer_inputs, rel_err

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
N_CASES = 40
MAX_WORK = 2.5e8  # S * (P + S) * Hq * D: keeps each oracle call to about a second


def _cases():
    rng = np.random.RandomState(20261202)
    out = []
    while len(out) < N_CASES:
        D = int(rng.choice([64, 128, 256]))
        Hkv = int(rng.choice([1, 2, 4, 8]))
        R = int(rng.choice([1, 2, 3, 4, 8]))
        S = int(rng.randint(2, 1200))
        P = 0 if rng.rand() < 0.5 else int(rng.randint(1, 3000))
        causal = bool(rng.rand() < 0.85)
        W = int(rng.randint(1, P + S + 1)) if rng.rand() < 0.25 else 0
        if S * (P + S) * Hkv * R * D > MAX_WORK:
            continue
        out.append((S, P, Hkv * R, Hkv, D, causal, W))
    return out


CASES = _cases()


@pytest.mark.parametrize("S,P,Hq,Hkv,D,causal,W", CASES,
                         ids=[f"S{c[0]}-P{c[1]}-{c[2]}q{c[3]}kv-d{c[4]}-{'c' if c[5] else 'nc'}-W{c[6]}" for c in CASES])
def test_random_prefill_shape(gpu, S, P, Hq, Hkv, D, causal, W):
    from spissa_amd.device import plan_attention

    cfg = gpu.KvAttentionConfig(S, Hq, Hkv, D, causal, W)
    plan = plan_attention(cfg, [P])
    print(f"[case] random prefill S={S} P={P} Hq={Hq} Hkv={Hkv} D={D} causal={causal} W={W} "
          f"plan: waves/block={plan['block_waves']} splits={plan['splits']} xcd={plan['xcd_group']} "
          f"workgroups={plan['workgroups']}", flush=True)
    q, k, v, pk, pv = layer_inputs(41, S + 7 * P + D, S, P, Hq, Hkv, D)
    cap = P + S + 3
    ref_cache = o.KvCache(Hkv, D, cap)
    dev_cache = gpu.KvCache(Hkv, D, cap)
    if P:
        ref_cache.append(pk, pv, P)
        dev_cache.append(pk, pv, P)
    ref = o.sdpa_with_cache(q, k, v, ref_cache, S, Hq, Hkv, D, causal, W)
    got = gpu.scaled_dot_product_attention_with_cache(q, k, v, dev_cache, cfg)
    assert np.all(np.isfinite(got))
    assert rel_err(got, ref) <= BF16_TOL
