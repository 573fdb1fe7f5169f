"""The Gemma 3 decode step on the device (spissa_gemma_decode_step_device):
QK-norm of q and the new key (ops.rs:159-179), Gemma RoPE (rotary.rs:137-186),
the q prescale (models/gemma/generate.rs:275), attention over the cache
(rotary.rs:335-415) and the append, in the decode step's two launches.

Bars: the output within 1e-4 of the oracle's prologue + attention (metric
max|gpu - ref| / max|ref|); the appended keys and values bit-identical to the
oracle's, and to the unfused device sequence (prologue, then the decode step
without RoPE), which is also compared on the output (within 1e-5: only q's
sum of squares is taken in another order).
"""
import numpy as np
import pytest

import oracle as o
from spissa_amd.synth import normal_f32, seed_for
from tests.helpers import assert_bitwise, layer_inputs, rel_err

pytestmark = pytest.mark.gpu

DECODE_TOL = 1e-4
EPS = 1e-6


def prescale_of(qpas: float, D: int) -> float:
    """(1 / sqrt(query_pre_attn_scalar)) * sqrt(head_dim) in f32, as generate.rs:275."""
    return float(np.float32(np.float32(1.0) / np.sqrt(np.float32(qpas))) * np.sqrt(np.float32(D)))


@pytest.mark.parametrize("name,B,Hq,Hkv,D,P,W,base,div,qpas", [
    ("gemma-1B global", 1, 4, 1, 256, 700, 0, 1e6, 8.0, 256.0),
    ("gemma-4B local W1024", 1, 8, 4, 256, 1500, 1024, 10000.0, 1.0, 256.0),
    ("prescale != 1", 1, 8, 4, 256, 300, 0, 10000.0, 1.0, 224.0),
    ("first token", 1, 4, 1, 256, 0, 0, 1e6, 8.0, 256.0),
    ("head_dim 128, three sequences", 3, 8, 2, 128, 513, 0, 10000.0, 1.0, 128.0),
    ("head_dim 64, window 1", 2, 6, 2, 64, 90, 1, 10000.0, 1.0, 64.0),
])
def test_gemma_decode_step_matches_prologue_attention_append(gpu, name, B, Hq, Hkv, D, P, W, base, div, qpas):
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session

    print(f"[case] gemma decode step {name} B={B} P={P}", flush=True)
    steps = 3
    pre = prescale_of(qpas, D)
    qn = normal_f32(seed_for(41, D, 0, "qnorm"), D, 1.0, 0.1)
    kn = normal_f32(seed_for(41, D, 0, "knorm"), D, 1.0, 0.1)
    s = Session(0)
    table = s.rope_table(_ffi.ROPE_GEMMA, D, base, div, max_positions=P + 7 * B + steps + 8)
    fused, unfused, refs, lens = [], [], [], []
    for b in range(B):
        n = P + 7 * b
        _, _, _, pk, pv = layer_inputs(40, b, 1, n, Hq, Hkv, D)
        dummy = np.zeros(max(1, n) * D, dtype=np.float32)
        if n:
            o.gemma_qk_prologue(dummy, pk, n, 1, Hkv, D, qn, kn, EPS, base, div, 0, qpas)  # past keys, normed
        c1, c2, r = s.kv_cache(Hkv, D, n + steps), s.kv_cache(Hkv, D, n + steps), o.KvCache(Hkv, D, n + steps)
        if n:
            for c in (c1, c2, r):
                c.append(pk, pv, n)
        fused.append(c1), unfused.append(c2), refs.append(r), lens.append(n)
    cfg = gpu.KvAttentionConfig(1, Hq, Hkv, D, True, W)
    dqn, dkn = torch.from_numpy(qn).cuda(), torch.from_numpy(kn).cuda()
    for t in range(steps):
        qs, ks, vs, wants = [], [], [], []
        for b in range(B):
            q, k, v, _, _ = layer_inputs(42, t, 1, 0, Hq, Hkv, D, sequence=b)
            rq, rk = q.copy(), k.copy()
            o.gemma_qk_prologue(rq, rk, 1, Hq, Hkv, D, qn, kn, EPS, base, div, refs[b].len(), qpas)
            wants.append(o.sdpa_with_cache(rq, rk, v, refs[b], 1, Hq, Hkv, D, True, W))
            refs[b].append(rk, v, 1)
            qs.append(q), ks.append(k), vs.append(v)
        q, k, v = (np.concatenate(x) for x in (qs, ks, vs))
        dq, dk, dv = (torch.from_numpy(x).cuda() for x in (q, k, v))
        out = torch.empty_like(dq)
        s.gemma_decode_step(table, dq, dk, dv, fused, cfg, dqn, dkn, EPS, pre, out)
        # the unfused sequence: the prologue in place on copies, then the step without RoPE
        uq, uk = dq.clone(), dk.clone()
        for b in range(B):
            s.gemma_qk_prologue(table, uq[b * Hq * D:(b + 1) * Hq * D], uk[b * Hkv * D:(b + 1) * Hkv * D], 1, Hq,
                                Hkv, D, dqn, dkn, EPS, lens[b] + t, pre)
        uout = torch.empty_like(dq)
        s.decode_step(None, uq, uk, dv, unfused, cfg, uout)
        s.sync()
        got = out.cpu().numpy().reshape(B, -1)
        ugot = uout.cpu().numpy().reshape(B, -1)
        for b in range(B):
            assert rel_err(got[b], wants[b]) <= DECODE_TOL, (t, b)
            assert rel_err(got[b], ugot[b]) <= 1e-5, (t, b)
        assert np.array_equal(dq.cpu().numpy(), q) and np.array_equal(dk.cpu().numpy(), k), "inputs are read-only"
    for b in range(B):
        assert fused[b].len() == lens[b] + steps
        assert_bitwise(fused[b].keys(), refs[b].keys(), f"seq {b} keys after fused steps")
        assert_bitwise(fused[b].values(), refs[b].values(), f"seq {b} values after fused steps")
        assert_bitwise(fused[b].keys(), unfused[b].keys(), f"seq {b} keys: fused vs unfused")


def test_gemma_decode_step_checks_its_arguments(gpu):
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session

    Hq, Hkv, D = 4, 1, 256
    s = Session(0)
    llama = s.rope_table(_ffi.ROPE_LLAMA, D, 10000.0, max_positions=64)
    gemma = s.rope_table(_ffi.ROPE_GEMMA, D, 10000.0, 1.0, max_positions=64)
    cache = s.kv_cache(Hkv, D, 4)
    cfg = gpu.KvAttentionConfig(1, Hq, Hkv, D, True)
    q = torch.zeros(Hq * D, device="cuda")
    k = torch.zeros(Hkv * D, device="cuda")
    w = torch.ones(D, device="cuda")
    out = torch.empty_like(q)
    with pytest.raises(gpu.ArgumentError):  # a llama table
        s.gemma_decode_step(llama, q, k, k, [cache], cfg, w, w, EPS, 1.0, out)
    with pytest.raises(gpu.ShapeError):  # query_len != 1
        s.gemma_decode_step(gemma, q, k, k, [cache], gpu.KvAttentionConfig(2, Hq, Hkv, D, True), w, w, EPS, 1.0,
                            out)
    assert cache.len() == 0
    for _ in range(4):
        s.gemma_decode_step(gemma, q, k, k, [cache], cfg, w, w, EPS, 1.0, out)
    with pytest.raises(gpu.ShapeError):  # the cache is full: checked before anything runs
        s.gemma_decode_step(gemma, q, k, k, [cache], cfg, w, w, EPS, 1.0, out)
    s.sync()
    assert cache.len() == 4
