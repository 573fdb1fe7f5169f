"""Seeded random decode batches against the CPU oracle.

The decode plan picks heads per block, rows per lane group, keys per split,
whether the new token gets a split of its own, and (above 16 sequences) the
number of launches, all from the shape of the call. This sweeps batches of
ragged cached lengths (empty caches included) across head dims 64/128/256,
GQA ratios 1-8 and windows, each sequence checked against the oracle at the
f32 decode bar: max|gpu - ref| / max|ref| <= 1e-4 per sequence.
"""
import numpy as np
import pytest

import oracle as o
from tests.helpers import layer_inputs, rel_err

pytestmark = pytest.mark.gpu

DECODE_TOL = 1e-4
N_CASES = 30
MAX_ROW_FLOATS = 2_000_000  # P * Hkv * D per sequence


def _cases():
    rng = np.random.RandomState(20261203)
    out = []
    while len(out) < N_CASES:
        D = int(rng.choice([64, 128, 256]))
        Hkv = int(rng.choice([1, 2, 4, 8]))
        R = int(rng.choice([1, 2, 3, 4, 8]))
        B = int(rng.choice([1, 1, 2, 5, 16, 19]))
        top = max(1, MAX_ROW_FLOATS // (Hkv * D))
        lens = [0 if rng.rand() < 0.1 else int(rng.randint(1, min(top, 9000))) for _ in range(B)]
        W = int(rng.randint(1, max(lens) + 2)) if rng.rand() < 0.3 else 0
        out.append((tuple(lens), Hkv * R, Hkv, D, W))
    return out


CASES = _cases()


@pytest.mark.parametrize("lens,Hq,Hkv,D,W", CASES,
                         ids=[f"B{len(c[0])}-max{max(c[0])}-{c[1]}q{c[2]}kv-d{c[3]}-W{c[4]}" for c in CASES])
def test_random_decode_batch(gpu, lens, Hq, Hkv, D, W):
    import torch

    from spissa_amd.device import Session, plan_attention

    cfg = gpu.KvAttentionConfig(1, Hq, Hkv, D, True, W)
    plan = plan_attention(cfg, list(lens))
    print(f"[case] random decode B={len(lens)} lens={list(lens)[:6]} Hq={Hq} Hkv={Hkv} D={D} W={W} "
          f"plan: path={plan['path']} heads/block={plan['heads_per_block']} keys/split={plan['keys_per_split']} "
          f"splits={plan['splits']} token_split={plan['token_split']}", flush=True)
    s = Session(0)
    caches, refs, qs, ks, vs = [], [], [], [], []
    for b, P in enumerate(lens):
        q, k, v, pk, pv = layer_inputs(43, D + P % 97, 1, P, Hq, Hkv, D, sequence=b)
        c = s.kv_cache(Hkv, D, P + 1)
        rc = o.KvCache(Hkv, D, P + 1)
        if P:
            c.append(pk, pv, P)
            rc.append(pk, pv, P)
        refs.append(o.sdpa_with_cache(q, k, v, rc, 1, Hq, Hkv, D, True, W))
        caches.append(c)
        qs.append(q), ks.append(k), vs.append(v)
    dq = torch.from_numpy(np.concatenate(qs)).cuda()
    dk = torch.from_numpy(np.concatenate(ks)).cuda()
    dv = torch.from_numpy(np.concatenate(vs)).cuda()
    out = torch.empty_like(dq)
    s.attention_decode_batch(dq, dk, dv, caches, cfg, out)
    s.sync()
    got = out.cpu().numpy().reshape(len(lens), -1)
    for b in range(len(lens)):
        assert rel_err(got[b], refs[b]) <= DECODE_TOL, (b, lens[b])
