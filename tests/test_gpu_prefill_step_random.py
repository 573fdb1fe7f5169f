"""Seeded random fused prefill steps: the append pass's shapes.

The fused step's first launch (RoPE, the optional Gemma QK-norm, the f32
cache rows and the bf16 operands) takes 64-row workgroups when that grid
gives every CU one, else 16-row ones, at head dims 64/128/256, with or
without the QK-norm and a RoPE table. This sweeps those choices over chunk
lengths and unaligned cache lengths, and checks each step on two bars:
  * output bitwise equal to the unfused device sequence on copies (RoPE in
    place, then the attention call and the append; for the Gemma form the QK
    prologue, then the plain step);
  * cache keys and values after the step bitwise equal to the oracle's RoPE
    (and QK-norm) and append (rotary.rs:226-256, ops.rs:159-179).
"""
import numpy as np
import pytest

import oracle as o
from tests.helpers import assert_bitwise, layer_inputs

pytestmark = pytest.mark.gpu

N_CASES = 24
CUS = 256  # MI355X


def wide_rows(S, P, Hq, Hkv, staged_q):
    """The launch's choice of 64-row workgroups (rope_norm.hip, launch_append_d), restated to label the cases."""
    pad_end = (P + S + 63) & ~63
    return (pad_end - (P & ~63)) // 64 * (2 * Hkv + (Hq if staged_q else 0)) >= CUS


def _cases():
    rng = np.random.RandomState(20261205)
    out = []
    while len(out) < N_CASES:
        D = int(rng.choice([64, 128, 256]))
        Hkv = int(rng.choice([1, 2, 4, 8]))
        R = int(rng.choice([1, 2, 3, 4]))
        S = int(rng.randint(2, 2600))
        P = 0 if rng.rand() < 0.4 else int(rng.randint(1, 2000))
        gemma = bool(rng.rand() < 0.4)
        kind = "gemma" if gemma else str(rng.choice(["llama", "gemma", "none"]))
        if S * (P + S) * Hkv * R * D > 6e9:
            continue
        out.append((S, P, Hkv * R, Hkv, D, gemma, kind))
    return out


CASES = _cases()


def _ids(c):
    S, P, Hq, Hkv, D, gemma, kind = c
    staged = gemma or D == 256
    return (f"S{S}-P{P}-{Hq}q{Hkv}kv-d{D}-{'gemma' if gemma else kind}-"
            f"{'64row' if wide_rows(S, P, Hq, Hkv, staged) else '16row'}")


@pytest.mark.parametrize("S,P,Hq,Hkv,D,gemma,kind", CASES, ids=[_ids(c) for c in CASES])
def test_random_prefill_step(gpu, S, P, Hq, Hkv, D, gemma, kind):
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig
    from spissa_amd.synth import normal_f32, seed_for

    print(f"[case] random prefill step {_ids((S, P, Hq, Hkv, D, gemma, kind))}", flush=True)
    base, div, eps = 10000.0, 1.0, 1e-6
    q, k, v, pk, pv = layer_inputs(44, D + S % 89, S, P, Hq, Hkv, D)
    s = Session(0)
    cfg = KvAttentionConfig(S, Hq, Hkv, D, True, 0)
    fused, plain = s.kv_cache(Hkv, D, P + S + 5), s.kv_cache(Hkv, D, P + S + 5)
    ref = o.KvCache(Hkv, D, P + S)
    dq, dk, dv = (torch.from_numpy(x).cuda() for x in (q, k, v))
    out_f = torch.full_like(dq, float("nan"))
    out_u = torch.full_like(dq, float("nan"))
    q2, k2 = dq.clone(), dk.clone()
    if gemma:
        qn = normal_f32(seed_for(44, D, S, "qnorm"), D, 1.0, 0.1)
        kn = normal_f32(seed_for(44, D, S, "knorm"), D, 1.0, 0.1)
        pre = float(np.float32(np.float32(1.0) / np.sqrt(np.float32(D))) * np.sqrt(np.float32(D)))
        if P:
            dummy = np.zeros(P * D, dtype=np.float32)
            o.gemma_qk_prologue(dummy, pk, P, 1, Hkv, D, qn, kn, eps, base, div, 0, D)
        table = s.rope_table(_ffi.ROPE_GEMMA, D, base, position_divisor=div, max_positions=P + S + 8)
        dqn, dkn = torch.from_numpy(qn).cuda(), torch.from_numpy(kn).cuda()
        for c in (fused, plain):
            if P:
                c.append(pk, pv, P)
        s.gemma_prefill_step(table, dq, dk, dv, fused, cfg, dqn, dkn, eps, pre, out_f)
        s.gemma_qk_prologue(table, q2, k2, S, Hq, Hkv, D, dqn, dkn, eps, P, pre)
        s.prefill_step(None, q2, k2, dv, plain, cfg, out_u)
        rq, rk = q.copy(), k.copy()
        o.gemma_qk_prologue(rq, rk, S, Hq, Hkv, D, qn, kn, eps, base, div, P, D)
    else:
        table = None
        if kind != "none":
            kid = _ffi.ROPE_LLAMA if kind == "llama" else _ffi.ROPE_GEMMA
            table = s.rope_table(kid, D, base, position_divisor=div, max_positions=P + S + 8)
        for c in (fused, plain):
            if P:
                c.append(pk, pv, P)
        s.prefill_step(table, dq, dk, dv, fused, cfg, out_f)
        if table is not None:
            s.rope_apply(table, q2, k2, S, Hq, Hkv, D, P)
        s.attention(q2, k2, dv, plain, cfg, out_u)
        s.append(plain, k2, dv, S)
        rq, rk = q.copy(), k.copy()
        if kind == "llama":
            o.apply_llama_rotary_inplace(rq, rk, Hq, Hkv, S, D, D, base, P)
        elif kind == "gemma":
            o.apply_gemma_rotary_inplace(rq, rk, Hq, Hkv, S, D, D, base, P, div)
    s.sync()
    assert np.array_equal(dq.cpu().numpy(), q) and np.array_equal(dk.cpu().numpy(), k), "inputs are read-only"
    assert_bitwise(out_f.cpu().numpy(), out_u.cpu().numpy(), "fused step vs the unfused sequence")
    if P:
        ref.append(pk, pv, P)
    ref.append(rk, v, S)
    assert fused.len() == P + S
    assert_bitwise(fused.keys(), ref.keys(), "keys after the step")
    assert_bitwise(fused.values(), ref.values(), "values after the step")
