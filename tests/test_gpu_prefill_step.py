"""The fused prefill step (spissa_prefill_step_device) against the unfused
device sequence and the CPU oracle.

The step is RoPE (rotary.rs:75-125 / 137-186) + attention over the cache and
the chunk (rotary.rs:335-415) + KvCache::append (rotary.rs:226-256) in two
launches. Bars:
  * output bitwise equal to the unfused device calls (rope_apply, attention,
    append) on the same inputs: both feed the MFMA kernel the same bf16
    operands, so the fusion may not change a single bit;
  * output <= 1e-2 (max|diff| / max|ref|) against the oracle's RoPE + SDPA;
  * cache rows (rotated keys, values) bitwise equal to the oracle's after the
    append.
"""
import numpy as np
import pytest

import oracle as o
from tests.helpers import assert_bitwise, layer_inputs, rel_err

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
DECODE_TOL = 1e-4


def _table(s, kind, D, base, divisor, positions):
    from spissa_amd import _ffi

    if kind is None:
        return None
    k = _ffi.ROPE_LLAMA if kind == "llama" else _ffi.ROPE_GEMMA
    return s.rope_table(k, D, base, position_divisor=divisor, max_positions=positions)


def _oracle_rope(kind, q, k, Hq, Hkv, S, D, base, divisor, P):
    q, k = q.copy(), k.copy()
    if kind == "llama":
        o.apply_llama_rotary_inplace(q, k, Hq, Hkv, S, D, D, base, P)
    elif kind == "gemma":
        o.apply_gemma_rotary_inplace(q, k, Hq, Hkv, S, D, D, base, P, divisor)
    return q, k


CASES = [  # name, S, P, Hq, Hkv, D, window, rope kind, base, divisor
    ("llama-3B shape prefill 512", 512, 0, 24, 8, 128, 0, "llama", 500000.0, 1.0),
    ("llama-3B chunk 100 on unaligned 333", 100, 333, 24, 8, 128, 0, "llama", 500000.0, 1.0),
    ("llama-1B shape chunk 200 on 64", 200, 64, 32, 8, 64, 0, "llama", 500000.0, 1.0),
    ("gemma-4B local chunk 128 on 1000 W1024", 128, 1000, 8, 4, 256, 1024, "gemma", 10000.0, 1.0),
    ("gemma-1B global prefill 300, divisor 8", 300, 0, 4, 1, 256, 0, "gemma", 1000000.0, 8.0),
    ("no RoPE, two tokens", 2, 5, 8, 2, 64, 0, None, 0.0, 1.0),
    # (64-row append workgroups: at least one per CU; the cases above take 16-row ones)
    ("8/8 heads, chunk 1000 on unaligned 37", 1000, 37, 8, 8, 128, 0, "llama", 500000.0, 1.0),
]


@pytest.mark.parametrize("name,S,P,Hq,Hkv,D,W,kind,base,div", CASES, ids=[c[0] for c in CASES])
def test_prefill_step_matches_unfused_sequence_and_oracle(gpu, name, S, P, Hq, Hkv, D, W, kind, base, div):
    import torch

    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig

    print(f"[case] prefill step {name}", flush=True)
    q, k, v, pk, pv = layer_inputs(40, S, S, P, Hq, Hkv, D)
    s = Session(0)
    table = _table(s, kind, D, base, div, P + S + 8)
    fused, plain = s.kv_cache(Hkv, D, P + S + 4), s.kv_cache(Hkv, D, P + S + 4)
    if P:
        fused.append(pk, pv, P)
        plain.append(pk, pv, P)
    dq, dk, dv = (torch.from_numpy(x).cuda() for x in (q, k, v))
    cfg = KvAttentionConfig(S, Hq, Hkv, D, True, W)
    out_f = torch.full_like(dq, float("nan"))
    s.prefill_step(table, dq, dk, dv, fused, cfg, out_f)
    # the unfused sequence on copies: RoPE in place, attention, append
    q2, k2 = dq.clone(), dk.clone()
    if table is not None:
        s.rope_apply(table, q2, k2, S, Hq, Hkv, D, P)
    out_p = torch.full_like(dq, float("nan"))
    s.attention(q2, k2, dv, plain, cfg, out_p)
    s.append(plain, k2, dv, S)
    # append-first order: the same attention over the cache that now holds the chunk
    out_c = torch.full_like(dq, float("nan"))
    if S > 1:
        s.attention_cached(q2, plain, cfg, out_c)
    s.sync()
    got, ref_dev = out_f.cpu().numpy(), out_p.cpu().numpy()
    assert np.array_equal(dq.cpu().numpy(), q) and np.array_equal(dk.cpu().numpy(), k), "inputs are read-only"
    assert_bitwise(got, ref_dev, "fused step vs unfused device sequence")
    if S > 1:
        assert_bitwise(out_c.cpu().numpy(), ref_dev, "append-first attention vs the unfused call")
    rq, rk = _oracle_rope(kind, q, k, Hq, Hkv, S, D, base, div, P)
    ref_cache = o.KvCache(Hkv, D, P + S)
    if P:
        ref_cache.append(pk, pv, P)
    want = o.sdpa_with_cache(rq, rk, v, ref_cache, S, Hq, Hkv, D, True, W)
    err = rel_err(got, want)
    print(f"[prefill step] {name}: rel err vs oracle {err:.2e}", flush=True)
    assert err <= BF16_TOL
    ref_cache.append(rk, v, S)
    assert fused.len() == P + S
    assert_bitwise(fused.keys(), ref_cache.keys(), "keys after the step")
    assert_bitwise(fused.values(), ref_cache.values(), "values after the step")


def test_prefill_steps_then_decode_steps_session(gpu):
    """A session the way a runtime drives it: a 64-token prompt step, a 40-token
    chunk step, then three decode steps, all on one cache; every output
    against the oracle and the cache bytes bitwise at the end."""
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig

    Hq, Hkv, D, theta = 24, 8, 128, 500000.0
    s = Session(0)
    table = s.rope_table(_ffi.ROPE_LLAMA, D, theta, max_positions=256)
    cache = s.kv_cache(Hkv, D, 200)
    ref = o.KvCache(Hkv, D, 200)
    for t, S in enumerate([64, 40, 1, 1, 1]):
        q, k, v, _, _ = layer_inputs(41, t, S, 0, Hq, Hkv, D)
        P = cache.len()
        rq, rk = _oracle_rope("llama", q, k, Hq, Hkv, S, D, theta, 1.0, P)
        want = o.sdpa_with_cache(rq, rk, v, ref, S, Hq, Hkv, D)
        ref.append(rk, v, S)
        dq, dk, dv = (torch.from_numpy(x).cuda() for x in (q, k, v))
        out = torch.empty_like(dq)
        s.prefill_step(table, dq, dk, dv, cache, KvAttentionConfig(S, Hq, Hkv, D, True), out)
        s.sync()
        assert rel_err(out.cpu().numpy(), want) <= (DECODE_TOL if S == 1 else BF16_TOL), (t, S)
    assert cache.len() == 107
    assert_bitwise(cache.keys(), ref.keys(), "keys")
    assert_bitwise(cache.values(), ref.values(), "values")


def test_prefill_step_checks_before_anything_runs(gpu):
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig

    s = Session(0)
    cache = s.kv_cache(2, 64, 10)
    x = torch.zeros(8 * 8 * 64, device="cuda")
    cache.append(np.zeros(5 * 128, np.float32), np.zeros(5 * 128, np.float32), 5)
    with pytest.raises(gpu.ShapeError):  # 8 rows do not fit a cache of 10 after 5
        s.prefill_step(None, x, x[:8 * 128], x[:8 * 128], cache, KvAttentionConfig(8, 8, 2, 64, True), x)
    assert cache.len() == 5
    with pytest.raises(gpu.ShapeError):  # head_dim 48 has no bf16 prefill
        s.prefill_step(None, x, x, x, s.kv_cache(2, 48, 16), KvAttentionConfig(4, 8, 2, 48, True), x)
    table = s.rope_table(_ffi.ROPE_LLAMA, 64, 10000.0, max_positions=6)
    with pytest.raises(gpu.ShapeError):  # positions 5..6 exceed a 6-position table
        s.prefill_step(table, x, x[:2 * 128], x[:2 * 128], cache, KvAttentionConfig(2, 8, 2, 64, True), x)
    assert cache.len() == 5


def test_append_first_attention_ignores_stale_rows_past_the_cache(gpu):
    """Rows beyond the cache's length that a longer earlier content left in
    the bf16 operands (NaN here) lie in the last key tile the kernel reads;
    the call zero-fills them, so they cannot reach the scores."""
    import torch

    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig

    Hq, Hkv, D, P, S = 8, 2, 128, 64, 36
    s = Session(0)
    q, k, v, pk, pv = layer_inputs(42, 0, S, P, Hq, Hkv, D)
    cache = s.kv_cache(Hkv, D, 256)
    junk = np.full(50 * Hkv * D, np.nan, dtype=np.float32)
    cache.append(pk, pv, P)
    # a first call creates the cache's bf16 operands; later appends update them
    first = torch.from_numpy(layer_inputs(42, 1, P, 0, Hq, Hkv, D)[0]).cuda()
    s.attention_cached(first, cache, KvAttentionConfig(P, Hq, Hkv, D, True), torch.empty_like(first))
    s.sync()
    cache.append(k, v, S)
    cache.append(junk, junk, 50)  # rows 100..149 (NaN), then rolled back
    cache.truncate(P + S)
    dq = torch.from_numpy(q).cuda()
    out = torch.empty_like(dq)
    s.attention_cached(dq, cache, KvAttentionConfig(S, Hq, Hkv, D, True), out)
    s.sync()
    ref = o.KvCache(Hkv, D, P)
    ref.append(pk, pv, P)
    want = o.sdpa_with_cache(q, k, v, ref, S, Hq, Hkv, D)
    got = out.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert rel_err(got, want) <= BF16_TOL


GEMMA_CASES = [  # name, S, P, Hq, Hkv, D, window, base, divisor, query_pre_attn_scalar
    ("gemma-1B global prefill 300, divisor 8", 300, 0, 4, 1, 256, 0, 1000000.0, 8.0, 256.0),
    ("gemma-4B local chunk 128 on 1000 W1024", 128, 1000, 8, 4, 256, 1024, 10000.0, 1.0, 256.0),
    ("prescale != 1, chunk 77 on 129", 77, 129, 8, 4, 256, 0, 10000.0, 1.0, 224.0),
    ("head_dim 128, 65 rows", 65, 0, 8, 2, 128, 0, 10000.0, 1.0, 128.0),
    ("head_dim 64, chunk 130 on 7", 130, 7, 6, 2, 64, 0, 10000.0, 1.0, 64.0),
    ("head_dim 64, 8/8 heads, chunk 700 on 37 (64-row append workgroups)", 700, 37, 8, 8, 64, 0, 10000.0, 1.0, 64.0),
]


@pytest.mark.parametrize("name,S,P,Hq,Hkv,D,W,base,div,qpas", GEMMA_CASES, ids=[c[0] for c in GEMMA_CASES])
def test_gemma_prefill_step_matches_prologue_then_step(gpu, name, S, P, Hq, Hkv, D, W, base, div, qpas):
    """spissa_gemma_prefill_step_device against the unfused device sequence
    (spissa_gemma_qk_prologue_device in place on copies, then the prefill step
    without RoPE): output and cache bitwise equal (the 1/rms pass sums the
    squares in index order, as the prologue does); against the oracle's
    prologue + SDPA (output <= 1e-2) and its cache after the append (bitwise)."""
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig
    from spissa_amd.synth import normal_f32, seed_for

    print(f"[case] gemma prefill step {name}", flush=True)
    eps = 1e-6
    pre = float(np.float32(np.float32(1.0) / np.sqrt(np.float32(qpas))) * np.sqrt(np.float32(D)))
    q, k, v, pk, pv = layer_inputs(52, D, S, P, Hq, Hkv, D)
    qn = normal_f32(seed_for(52, D, 0, "qnorm"), D, 1.0, 0.1)
    kn = normal_f32(seed_for(52, D, 0, "knorm"), D, 1.0, 0.1)
    if P:
        dummy = np.zeros(P * D, dtype=np.float32)
        o.gemma_qk_prologue(dummy, pk, P, 1, Hkv, D, qn, kn, eps, base, div, 0, qpas)
    ref = o.KvCache(Hkv, D, P + S)
    if P:
        ref.append(pk, pv, P)
    rq, rk = q.copy(), k.copy()
    o.gemma_qk_prologue(rq, rk, S, Hq, Hkv, D, qn, kn, eps, base, div, P, qpas)
    want = o.sdpa_with_cache(rq, rk, v, ref, S, Hq, Hkv, D, True, W)
    ref.append(rk, v, S)

    s = Session(0)
    table = s.rope_table(_ffi.ROPE_GEMMA, D, base, position_divisor=div, max_positions=P + S + 8)
    fused, unfused = s.kv_cache(Hkv, D, P + S), s.kv_cache(Hkv, D, P + S)
    if P:
        fused.append(pk, pv, P)
        unfused.append(pk, pv, P)
    cfg = KvAttentionConfig(S, Hq, Hkv, D, True, W)
    dq, dk, dv, dqn, dkn = (torch.from_numpy(x).cuda() for x in (q, k, v, qn, kn))
    out = torch.empty_like(dq)
    s.gemma_prefill_step(table, dq, dk, dv, fused, cfg, dqn, dkn, eps, pre, out)
    uq, uk = dq.clone(), dk.clone()
    s.gemma_qk_prologue(table, uq, uk, S, Hq, Hkv, D, dqn, dkn, eps, P, pre)
    uout = torch.empty_like(dq)
    s.prefill_step(None, uq, uk, dv, unfused, cfg, uout)
    s.sync()
    got = out.cpu().numpy()
    assert np.array_equal(dq.cpu().numpy(), q) and np.array_equal(dk.cpu().numpy(), k), "inputs are read-only"
    assert_bitwise(got, uout.cpu().numpy(), "output: fused vs prologue + step")
    assert_bitwise(fused.keys(), unfused.keys(), "keys: fused vs prologue + step")
    assert rel_err(got, want) <= BF16_TOL
    assert fused.len() == P + S
    assert_bitwise(fused.keys(), ref.keys(), "keys against the oracle")
    assert_bitwise(fused.values(), ref.values(), "values against the oracle")


def test_gemma_prefill_step_checks_its_arguments(gpu):
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig

    Hq, Hkv, D, S = 4, 1, 256, 8
    s = Session(0)
    llama = s.rope_table(_ffi.ROPE_LLAMA, D, 10000.0, max_positions=64)
    gemma = s.rope_table(_ffi.ROPE_GEMMA, D, 10000.0, position_divisor=1.0, max_positions=64)
    cache = s.kv_cache(Hkv, D, 12)
    cfg = KvAttentionConfig(S, Hq, Hkv, D, True)
    q = torch.zeros(S * Hq * D, device="cuda")
    k = torch.zeros(S * Hkv * D, device="cuda")
    w = torch.ones(D, device="cuda")
    out = torch.empty_like(q)
    with pytest.raises(gpu.ArgumentError):  # a llama table
        s.gemma_prefill_step(llama, q, k, k, cache, cfg, w, w, 1e-6, 1.0, out)
    s.gemma_prefill_step(gemma, q, k, k, cache, cfg, w, w, 1e-6, 1.0, out)
    with pytest.raises(gpu.ShapeError):  # 8 more rows exceed the capacity of 12: nothing runs
        s.gemma_prefill_step(gemma, q, k, k, cache, cfg, w, w, 1e-6, 1.0, out)
    s.sync()
    assert cache.len() == 8
