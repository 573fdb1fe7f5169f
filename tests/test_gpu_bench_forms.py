"""GPU parity of the exact launch forms bench.py times, at the bench's shapes.

Each test calls the entry point the bench times, with the bench's geometry
(heads, head_dim, cached and new rows, window, RoPE base and divisor), and
compares with the CPU oracle:
  * Llama-3.2-3B prefill of 4096 tokens through spissa_prefill_step_device
    (RoPE + append + attention) and spissa_attention_cached_device (the step's
    attention launch alone over the cache holding the prompt);
  * the Gemma prefill step (spissa_gemma_prefill_step_device): Gemma-3-1B
    4096 tokens, global and W512, and the Gemma-3-4B chunk of 128 tokens on
    16384 cached ones, global and W1024;
  * the fused decode steps: Llama-3.2-3B at 8192 cached tokens, batch 1
    (spissa_decode_step_device, the headline launch), and the Gemma decode
    step (spissa_gemma_decode_step_device) at 32768 keys (Gemma-3-1B, global
    and W512) and at 16512 keys (Gemma-3-4B after the chunk, global and W1024).
Prefill outputs are checked on blocks of query rows spread over the call (the
first, the last and those between), each as a chunked oracle call with the
earlier rows in the cache; decode outputs whole. Appended cache rows (the
normed and rotated keys, the values) are bitwise the oracle's.
Tolerances: bf16 prefill 1e-2, f32 decode 1e-4 (max|diff| / max|ref|).
The QK-norm weights are N(1, 0.1) multipliers, eps 1e-6, q prescale 1.0
(query_pre_attn_scalar = head_dim), as models/gemma/generate.rs:232-278 uses
them for these models.
"""
import numpy as np
import pytest

import oracle as o
from spissa_amd.synth import normal_f32, seed_for
from tests.helpers import assert_bitwise, layer_inputs, rel_err
from tests.test_gpu_scale import oracle_blocks, spaced_blocks

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
DECODE_TOL = 1e-4
EPS = 1e-6


def _rows(a, width, lo, hi):
    return np.asarray(a).reshape(-1, width)[lo:hi].ravel()


def _gemma_table(s, D, base, divisor, positions):
    from spissa_amd import _ffi

    return s.rope_table(_ffi.ROPE_GEMMA, D, base, position_divisor=divisor, max_positions=positions)


def _norm_weights(config, layer, D):
    return (normal_f32(seed_for(config, layer, 0, "qnorm"), D, 1.0, 0.1),
            normal_f32(seed_for(config, layer, 0, "knorm"), D, 1.0, 0.1))


def test_llama3b_prefill_step_and_cached_attention_at_4096(gpu):
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig

    print("[case] llama-3B prefill step + cached attention, 4096 x 24/8 x 128", flush=True)
    S, Hq, Hkv, D, theta = 4096, 24, 8, 128, 500000.0
    q, k, v, _, _ = layer_inputs(41, 0, S, 0, Hq, Hkv, D)
    rq, rk = q.copy(), k.copy()
    o.apply_llama_rotary_inplace(rq, rk, Hq, Hkv, S, D, D, theta, 0)
    blocks = spaced_blocks(S, 32)
    refs = oracle_blocks(rq, rk, v, Hq, Hkv, D, blocks)

    s = Session(0)
    table = s.rope_table(_ffi.ROPE_LLAMA, D, theta, max_positions=S + 64)
    cache = s.kv_cache(Hkv, D, S)
    cfg = KvAttentionConfig(S, Hq, Hkv, D, True)
    dq, dk, dv = (torch.from_numpy(x).cuda() for x in (q, k, v))
    out = torch.full_like(dq, float("nan"))
    s.prefill_step(table, dq, dk, dv, cache, cfg, out)
    s.sync()
    step = out.cpu().numpy()
    assert np.all(np.isfinite(step))
    for (lo, hi), ref in zip(blocks, refs):
        assert rel_err(_rows(step, Hq * D, lo, hi), ref) <= BF16_TOL, ("prefill step", lo, hi)
    assert cache.len() == S
    assert_bitwise(cache.keys(), rk, "rotated keys appended by the step")
    assert_bitwise(cache.values(), v, "values appended by the step")

    # the step's attention launch alone, over the cache that holds the prompt
    drq = torch.from_numpy(rq).cuda()
    out2 = torch.full_like(dq, float("nan"))
    s.attention_cached(drq, cache, cfg, out2)
    s.sync()
    cached = out2.cpu().numpy()
    for (lo, hi), ref in zip(blocks, refs):
        assert rel_err(_rows(cached, Hq * D, lo, hi), ref) <= BF16_TOL, ("cached attention", lo, hi)
    assert rel_err(cached, step) <= BF16_TOL


GEMMA_PREFILL = [  # name, S, P, Hq, Hkv, window, base, divisor, block rows, blocks
    ("gemma-1B prefill 4096 global", 4096, 0, 4, 1, 0, 1000000.0, 8.0, 32, 10),
    ("gemma-1B prefill 4096 local W512", 4096, 0, 4, 1, 512, 10000.0, 1.0, 32, 10),
    ("gemma-4B chunk 128 on 16384 global", 128, 16384, 8, 4, 0, 1000000.0, 8.0, 16, 8),
    ("gemma-4B chunk 128 on 16384 local W1024", 128, 16384, 8, 4, 1024, 10000.0, 1.0, 16, 8),
]


@pytest.mark.parametrize("name,S,P,Hq,Hkv,W,base,div,rows,count", GEMMA_PREFILL, ids=[c[0] for c in GEMMA_PREFILL])
def test_gemma_prefill_step_at_bench_shapes(gpu, name, S, P, Hq, Hkv, W, base, div, rows, count):
    import torch

    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig

    print(f"[case] gemma prefill step {name}", flush=True)
    D = 256
    q, k, v, pk, pv = layer_inputs(42, W + P, S, P, Hq, Hkv, D)
    qn, kn = _norm_weights(42, W + P, D)
    rq, rk = q.copy(), k.copy()
    o.gemma_qk_prologue(rq, rk, S, Hq, Hkv, D, qn, kn, EPS, base, div, P, float(D))
    blocks = spaced_blocks(S, rows, count)
    refs = oracle_blocks(rq, rk, v, Hq, Hkv, D, blocks, W, past_k=pk if P else None, past_v=pv if P else None)

    s = Session(0)
    table = _gemma_table(s, D, base, div, P + S + 64)
    cache = s.kv_cache(Hkv, D, P + S)
    if P:
        cache.append(pk, pv, P)
    cfg = KvAttentionConfig(S, Hq, Hkv, D, True, W)
    dq, dk, dv, dqn, dkn = (torch.from_numpy(x).cuda() for x in (q, k, v, qn, kn))
    out = torch.full_like(dq, float("nan"))
    s.gemma_prefill_step(table, dq, dk, dv, cache, cfg, dqn, dkn, EPS, 1.0, out)
    s.sync()
    got = out.cpu().numpy()
    assert np.all(np.isfinite(got))
    worst = 0.0
    for (lo, hi), ref in zip(blocks, refs):
        err = rel_err(_rows(got, Hq * D, lo, hi), ref)
        worst = max(worst, err)
        assert err <= BF16_TOL, (lo, hi)
    print(f"[gemma prefill] {name}: worst block rel err {worst:.2e}", flush=True)
    assert cache.len() == P + S
    w = Hkv * D
    assert_bitwise(cache.keys()[P * w:], rk, "normed and rotated keys appended by the step")
    assert_bitwise(cache.values()[P * w:], v, "values appended by the step")
    if P:
        assert_bitwise(cache.keys()[:P * w], pk, "cached keys untouched")


def test_llama3b_decode_step_at_8192_batch1(gpu):
    """The headline launch: one fused decode step (RoPE, split-K attention
    with the new token as split 0, append) per layer at 8192 cached tokens."""
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session, plan_attention
    from spissa_amd.rotary import KvAttentionConfig

    print("[case] llama-3B fused decode step @8192 batch 1", flush=True)
    Hq, Hkv, D, P, theta = 24, 8, 128, 8192, 500000.0
    cfg = KvAttentionConfig(1, Hq, Hkv, D, True)
    plan = plan_attention(cfg, [P])
    assert plan["token_split"] == 1 and plan["splits"] > 32 and plan["workgroups"] <= 512  # the form the bench times
    s = Session(0)
    table = s.rope_table(_ffi.ROPE_LLAMA, D, theta, max_positions=P + 64)
    for layer in range(3):
        q, k, v, pk, pv = layer_inputs(43, layer, 1, P, Hq, Hkv, D)
        cache = s.kv_cache(Hkv, D, P + 1)
        cache.append(pk, pv, P)
        ref = o.KvCache(Hkv, D, P + 1)
        ref.append(pk, pv, P)
        rq, rk = q.copy(), k.copy()
        o.apply_llama_rotary_inplace(rq, rk, Hq, Hkv, 1, D, D, theta, P)
        want = o.sdpa_with_cache(rq, rk, v, ref, 1, Hq, Hkv, D)
        dq, dk, dv = (torch.from_numpy(x).cuda() for x in (q, k, v))
        out = torch.full_like(dq, float("nan"))
        s.decode_step(table, dq, dk, dv, [cache], cfg, out)
        s.sync()
        err = rel_err(out.cpu().numpy(), want)
        print(f"[decode] layer {layer}: rel err {err:.2e}", flush=True)
        assert err <= DECODE_TOL, layer
        assert cache.len() == P + 1
        assert_bitwise(cache.keys()[P * Hkv * D:], rk, "appended rotated key")
        assert_bitwise(cache.values()[P * Hkv * D:], v, "appended value")


GEMMA_DECODE = [  # name, P, Hq, Hkv, window, base, divisor
    ("gemma-1B @32768 global", 32768, 4, 1, 0, 1000000.0, 8.0),
    ("gemma-1B @32768 local W512", 32768, 4, 1, 512, 10000.0, 1.0),
    ("gemma-4B @16512 global", 16512, 8, 4, 0, 1000000.0, 8.0),
    ("gemma-4B @16512 local W1024", 16512, 8, 4, 1024, 10000.0, 1.0),
]


@pytest.mark.parametrize("name,P,Hq,Hkv,W,base,div", GEMMA_DECODE, ids=[c[0] for c in GEMMA_DECODE])
def test_gemma_decode_step_at_bench_shapes(gpu, name, P, Hq, Hkv, W, base, div):
    import torch

    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig

    print(f"[case] gemma fused decode step {name}", flush=True)
    D = 256
    q, k, v, pk, pv = layer_inputs(44, W + P, 1, P, Hq, Hkv, D)
    qn, kn = _norm_weights(44, W + P, D)
    rq, rk = q.copy(), k.copy()
    o.gemma_qk_prologue(rq, rk, 1, Hq, Hkv, D, qn, kn, EPS, base, div, P, float(D))
    ref = o.KvCache(Hkv, D, P + 1)
    ref.append(pk, pv, P)
    want = o.sdpa_with_cache(rq, rk, v, ref, 1, Hq, Hkv, D, True, W)

    s = Session(0)
    table = _gemma_table(s, D, base, div, P + 64)
    cache = s.kv_cache(Hkv, D, P + 1)
    cache.append(pk, pv, P)
    cfg = KvAttentionConfig(1, Hq, Hkv, D, True, W)
    dq, dk, dv, dqn, dkn = (torch.from_numpy(x).cuda() for x in (q, k, v, qn, kn))
    out = torch.full_like(dq, float("nan"))
    s.gemma_decode_step(table, dq, dk, dv, [cache], cfg, dqn, dkn, EPS, 1.0, out)
    s.sync()
    err = rel_err(out.cpu().numpy(), want)
    print(f"[gemma decode] {name}: rel err {err:.2e}", flush=True)
    assert err <= DECODE_TOL
    assert cache.len() == P + 1
    assert_bitwise(cache.keys()[P * Hkv * D:], rk, "appended normed and rotated key")
    assert_bitwise(cache.values()[P * Hkv * D:], v, "appended value")
