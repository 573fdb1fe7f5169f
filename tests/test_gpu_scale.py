"""GPU parity at the BASELINE configurations' full sizes.

The oracle is C, one call per thread; at full size it is run only where it
finishes in seconds:
  * blocks of a prefill's query rows spread evenly over the prompt (the first,
    the last and eight between), as chunked calls: a call with the earlier
    rows in the cache computes those rows exactly as the one-shot call does
    (same keys, same loop order, rotary.rs:335-415);
  * single-token decode (tens of milliseconds per call);
  * cache contents, which are bitwise.
Size-independent properties cover the rest: the bf16-MFMA prefill against the
device's f32 path on every row, the cache bytes after thousands of appends,
and the decode of every step of a prefill-then-decode session.
Tolerances: f32 decode 1e-4, bf16 prefill 1e-2 (max|diff| / max|ref|).
"""
import numpy as np
import pytest

import oracle as o
from tests.helpers import assert_bitwise, layer_inputs, rel_err

pytestmark = pytest.mark.gpu

DECODE_TOL = 1e-4
BF16_TOL = 1e-2


def _torch():
    import torch

    return torch


def _rows(a, S, width, lo, hi):
    return a.reshape(S, width)[lo:hi].ravel()


def oracle_rows(q, k, v, S, Hq, Hkv, D, lo, hi, window=0, past_k=None, past_v=None):
    """Oracle output rows [lo, hi) of a causal call over S new rows (plus optional past rows)."""
    P = 0 if past_k is None else past_k.size // (Hkv * D)
    w, wq = Hkv * D, Hq * D
    cache = o.KvCache(Hkv, D, P + hi)
    if P:
        cache.append(past_k, past_v, P)
    if lo:
        cache.append(k[:lo * w].copy(), v[:lo * w].copy(), lo)
    return o.sdpa_with_cache(q[lo * wq:hi * wq].copy(), k[lo * w:hi * w].copy(), v[lo * w:hi * w].copy(), cache,
                             hi - lo, Hq, Hkv, D, True, window)


def spaced_blocks(S, rows, count=10):
    """`count` blocks of `rows` query rows spread evenly over [0, S), both ends included."""
    return [(lo, lo + rows) for lo in sorted({(i * (S - rows)) // (count - 1) for i in range(count)})]


def oracle_blocks(q, k, v, Hq, Hkv, D, blocks, window=0, past_k=None, past_v=None, threads=16):
    """Oracle output rows [lo, hi) of a causal call for every block, each as a
    chunked call (the rows before lo in the cache), run on `threads` threads."""
    P = 0 if past_k is None else past_k.size // (Hkv * D)
    w, wq = Hkv * D, Hq * D
    units = []
    for lo, hi in blocks:
        cache = o.KvCache(Hkv, D, P + hi)
        if P:
            cache.append(past_k, past_v, P)
        if lo:
            cache.append(k[:lo * w].copy(), v[:lo * w].copy(), lo)
        units.append((q[lo * wq:hi * wq].copy(), k[lo * w:hi * w].copy(), v[lo * w:hi * w].copy(), cache))
    rows = blocks[0][1] - blocks[0][0]
    assert all(hi - lo == rows for lo, hi in blocks)
    return o.sdpa_many(units, (rows, Hq, Hkv, D, 1, window), threads)


def device_attention(s, q, k, v, cache, S, Hq, Hkv, D, window=0, precision=None):
    torch = _torch()
    from spissa_amd.rotary import KvAttentionConfig

    if precision is not None:
        s.set_prefill_precision(precision)
    dq, dk, dv = (torch.from_numpy(x).cuda() for x in (q, k, v))
    out = torch.empty_like(dq)
    s.attention(dq, dk, dv, cache, KvAttentionConfig(S, Hq, Hkv, D, True, window), out)
    s.sync()
    return out.cpu().numpy()


@pytest.mark.parametrize("name,S,Hq,Hkv,D,window", [
    ("cfg3a llama-3B prefill 4096", 4096, 24, 8, 128, 0),
    ("cfg2 llama-1B prefill 2048", 2048, 32, 8, 64, 0),
    ("cfg4 gemma-1B global prefill 4096", 4096, 4, 1, 256, 0),
    ("cfg4 gemma-1B local W512 prefill 4096", 4096, 4, 1, 256, 512),
])
def test_full_prefill_rows_and_f32_cross_check(gpu, name, S, Hq, Hkv, D, window):
    from spissa_amd import _ffi
    from spissa_amd.device import Session

    print(f"[case] full prefill {name}", flush=True)
    q, k, v, _, _ = layer_inputs(30, S % 7, S, 0, Hq, Hkv, D)
    s = Session(0)
    got = device_attention(s, q, k, v, None, S, Hq, Hkv, D, window)
    f32 = device_attention(s, q, k, v, None, S, Hq, Hkv, D, window, precision=_ffi.PREFILL_F32)
    s.set_prefill_precision(_ffi.PREFILL_BF16)
    assert np.all(np.isfinite(got))
    assert rel_err(got, f32) <= BF16_TOL, "bf16 prefill vs the device f32 path, all rows"
    wq = Hq * D
    # ten 32-row query blocks spread over the prompt (first, last and eight
    # between, at offsets that are not tile-aligned), each against the oracle
    blocks = spaced_blocks(S, 32)
    refs = oracle_blocks(q, k, v, Hq, Hkv, D, blocks, window)
    for (lo, hi), ref in zip(blocks, refs):
        assert rel_err(_rows(got, S, wq, lo, hi), ref) <= BF16_TOL, (lo, hi)
        assert rel_err(_rows(f32, S, wq, lo, hi), ref) <= DECODE_TOL, ("f32 path", lo, hi)


def test_cfg3b_batch16_decode_at_8192_fused(gpu):
    """Llama-3.2-3B decode, 16 sequences of 8192 cached tokens, one fused step."""
    torch = _torch()
    from spissa_amd import _ffi
    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig

    print("[case] cfg3b batch-16 fused decode @8192", flush=True)
    B, Hq, Hkv, D, P, theta = 16, 24, 8, 128, 8192, 500000.0
    s = Session(0)
    table = s.rope_table(_ffi.ROPE_LLAMA, D, theta, max_positions=P + 8)
    caches, refs, qs, ks, vs = [], [], [], [], []
    for b in range(B):
        q, k, v, pk, pv = layer_inputs(31, 0, 1, P, Hq, Hkv, D, sequence=b)
        c = s.kv_cache(Hkv, D, P + 1)
        c.append(pk, pv, P)
        rc = o.KvCache(Hkv, D, P + 1)
        rc.append(pk, pv, P)
        caches.append(c)
        refs.append(rc)
        qs.append(q)
        ks.append(k)
        vs.append(v)
    dq, dk, dv = (torch.from_numpy(np.concatenate(x)).cuda() for x in (qs, ks, vs))
    out = torch.empty_like(dq)
    s.decode_step(table, dq, dk, dv, caches, KvAttentionConfig(1, Hq, Hkv, D, True), out)
    s.sync()
    got = out.cpu().numpy().reshape(B, -1)
    units = []
    for b in range(B):
        rq, rk = qs[b].copy(), ks[b].copy()
        o.apply_llama_rotary_inplace(rq, rk, Hq, Hkv, 1, D, D, theta, P)
        units.append((rq, rk, vs[b], refs[b]))
    want = o.sdpa_many(units, (1, Hq, Hkv, D, 1, 0), 16)
    for b in range(B):
        assert rel_err(got[b], want[b]) <= DECODE_TOL, b
        refs[b].append(units[b][1], vs[b], 1)
        assert caches[b].len() == P + 1
    # appended rows (rotated keys) bitwise, read back through the drop-in accessor
    for b in (0, B - 1):
        assert_bitwise(caches[b].keys()[P * Hkv * D:], refs[b].keys()[P * Hkv * D:], f"seq {b} appended key")
        assert_bitwise(caches[b].values(), refs[b].values(), f"seq {b} values")


def test_cfg2_prefill_2048_then_128_decode_steps(gpu):
    """Llama-3.2-1B: prefill 2048 (RoPE, attention, append), then 128 fused decode steps."""
    torch = _torch()
    from spissa_amd import _ffi
    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig

    print("[case] cfg2 prefill 2048 + 128 decode", flush=True)
    Hq, Hkv, D, S0, steps, theta = 32, 8, 64, 2048, 128, 500000.0
    s = Session(0)
    table = s.rope_table(_ffi.ROPE_LLAMA, D, theta, max_positions=S0 + steps + 8)
    cache = s.kv_cache(Hkv, D, S0 + steps)
    ref = o.KvCache(Hkv, D, S0 + steps)
    q, k, v, _, _ = layer_inputs(32, 3, S0, 0, Hq, Hkv, D)
    rq, rk = q.copy(), k.copy()
    o.apply_llama_rotary_inplace(rq, rk, Hq, Hkv, S0, D, D, theta, 0)
    dq, dk, dv = (torch.from_numpy(x).cuda() for x in (q, k, v))
    s.rope_apply(table, dq, dk, S0, Hq, Hkv, D, 0)
    assert_bitwise(dq.cpu().numpy(), rq, "prompt q RoPE")
    out = torch.empty_like(dq)
    s.attention(dq, dk, dv, cache, KvAttentionConfig(S0, Hq, Hkv, D, True), out)
    s.append(cache, dk, dv, S0)
    s.sync()
    ref.append(rk, v, S0)
    want_tail = oracle_rows(rq, rk, v, S0, Hq, Hkv, D, S0 - 32, S0)
    assert rel_err(_rows(out.cpu().numpy(), S0, Hq * D, S0 - 32, S0), want_tail) <= BF16_TOL
    cfg = KvAttentionConfig(1, Hq, Hkv, D, True)
    worst = 0.0
    for t in range(steps):
        q1, k1, v1, _, _ = layer_inputs(33, t, 1, 0, Hq, Hkv, D)
        rq1, rk1 = q1.copy(), k1.copy()
        o.apply_llama_rotary_inplace(rq1, rk1, Hq, Hkv, 1, D, D, theta, S0 + t)
        want = o.sdpa_with_cache(rq1, rk1, v1, ref, 1, Hq, Hkv, D)
        ref.append(rk1, v1, 1)
        d1 = [torch.from_numpy(x).cuda() for x in (q1, k1, v1)]
        o1 = torch.empty_like(d1[0])
        s.decode_step(table, d1[0], d1[1], d1[2], [cache], cfg, o1)
        s.sync()
        worst = max(worst, rel_err(o1.cpu().numpy(), want))
    assert worst <= DECODE_TOL
    assert cache.len() == S0 + steps
    assert_bitwise(cache.keys(), ref.keys(), "keys after prefill + 128 steps")
    assert_bitwise(cache.values(), ref.values(), "values after prefill + 128 steps")


def test_cfg5_chunk_128_on_16384_then_decode(gpu):
    """Gemma-3-4B resident cache: 16384 cached tokens, a 128-token chunk (global
    and local W1024 layers), then all 256 decode steps of the workload
    appending to the same cache, with the cache bytes checked bitwise."""
    torch = _torch()
    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig

    print("[case] cfg5 chunk 128 on 16384 + 256 decode steps", flush=True)
    Hq, Hkv, D, P, S, steps = 8, 4, 256, 16384, 128, 256
    s = Session(0)
    for window in (0, 1024):
        q, k, v, pk, pv = layer_inputs(34, window, S, P, Hq, Hkv, D)
        cache = s.kv_cache(Hkv, D, P + S + steps)
        cache.append(pk, pv, P)
        got = device_attention(s, q, k, v, cache, S, Hq, Hkv, D, window)
        blocks = spaced_blocks(S, 16, count=8)
        refs = oracle_blocks(q, k, v, Hq, Hkv, D, blocks, window, past_k=pk, past_v=pv)
        for (lo, hi), ref in zip(blocks, refs):
            assert rel_err(_rows(got, S, Hq * D, lo, hi), ref) <= BF16_TOL, (window, lo, hi)
        cache.append(k, v, S)
        ref_cache = o.KvCache(Hkv, D, P + S + steps)
        ref_cache.append(pk, pv, P)
        ref_cache.append(k, v, S)
        cfg = KvAttentionConfig(1, Hq, Hkv, D, True, window)
        for t in range(steps):
            q1, k1, v1, _, _ = layer_inputs(35, t, 1, 0, Hq, Hkv, D, sequence=window)
            want = o.sdpa_with_cache(q1, k1, v1, ref_cache, 1, Hq, Hkv, D, True, window)
            ref_cache.append(k1, v1, 1)
            d1 = [torch.from_numpy(x).cuda() for x in (q1, k1, v1)]
            o1 = torch.empty_like(d1[0])
            s.decode_step(None, d1[0], d1[1], d1[2], [cache], cfg, o1)
            s.sync()
            assert rel_err(o1.cpu().numpy(), want) <= DECODE_TOL, (window, t)
        assert_bitwise(cache.keys(), ref_cache.keys(), f"keys W={window}")
        assert_bitwise(cache.values(), ref_cache.values(), f"values W={window}")


def test_cache_over_4GiB_per_buffer_uses_generic_decode(gpu):
    """A cache whose buffers exceed the split kernel's 32-bit offsets: the
    attention call falls back to the f32 SIMT kernel; the fused step refuses."""
    torch = _torch()
    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig

    print("[case] >4 GiB cache buffers", flush=True)
    Hq, Hkv, D, P = 16, 8, 128, 1000
    max_seq = (1 << 32) // (Hkv * D * 4) + 64  # one buffer just over 4 GiB
    s = Session(0)
    cache = s.kv_cache(Hkv, D, max_seq)
    q, k, v, pk, pv = layer_inputs(36, 0, 1, P, Hq, Hkv, D)
    cache.append(pk, pv, P)
    ref = o.KvCache(Hkv, D, P + 1)
    ref.append(pk, pv, P)
    got = device_attention(s, q, k, v, cache, 1, Hq, Hkv, D)
    want = o.sdpa_with_cache(q, k, v, ref, 1, Hq, Hkv, D)
    assert rel_err(got, want) <= DECODE_TOL
    d1 = [torch.from_numpy(x).cuda() for x in (q, k, v)]
    with pytest.raises(gpu.ShapeError):
        s.decode_step(None, d1[0], d1[1], d1[2], [cache], KvAttentionConfig(1, Hq, Hkv, D, True),
                      torch.empty_like(d1[0]))
    assert cache.len() == P
    del cache


@pytest.mark.parametrize("name,base,divisor,window", [
    ("global theta 1e6 divisor 8", 1000000.0, 8.0, 0),
    ("local theta 1e4 W512", 10000.0, 1.0, 512),
])
def test_cfg4_gemma_qk_norm_rope_decode_at_32768(gpu, name, base, divisor, window):
    """Gemma-3-1B decode at 32768 cached tokens with the whole layer prologue
    (models/gemma/generate.rs:232-295): QK-norm of the new q and k rows
    (ops.rs:159-179), Gemma RoPE at position 32768 (rotary.rs:137-186), the
    x1.0 prescale, attention over the cache (global, or the W512 window), then
    the append. The cached keys went through the same prologue at their own
    positions. Prologue bitwise, output <= 1e-4 against the oracle."""
    torch = _torch()
    from spissa_amd import _ffi
    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig
    from spissa_amd.synth import normal_f32, seed_for

    print(f"[case] cfg4 gemma-1B QK-norm + RoPE + decode @32768 {name}", flush=True)
    Hq, Hkv, D, P, eps = 4, 1, 256, 32768, 1e-6
    q, k, v, pk, pv = layer_inputs(37, window, 1, P, Hq, Hkv, D)
    qn = normal_f32(seed_for(37, window, 0, "qnorm"), D, 1.0, 0.1)
    kn = normal_f32(seed_for(37, window, 0, "knorm"), D, 1.0, 0.1)
    # cached keys: normed and rotated at positions 0..P-1 (the past prologues)
    dummy = np.zeros(P * D, dtype=np.float32)
    o.gemma_qk_prologue(dummy, pk, P, 1, Hkv, D, qn, kn, eps, base, divisor, 0, float(D))
    ref_cache = o.KvCache(Hkv, D, P + 1)
    ref_cache.append(pk, pv, P)
    rq, rk = q.copy(), k.copy()
    o.gemma_qk_prologue(rq, rk, 1, Hq, Hkv, D, qn, kn, eps, base, divisor, P, float(D))
    want = o.sdpa_with_cache(rq, rk, v, ref_cache, 1, Hq, Hkv, D, True, window)
    ref_cache.append(rk, v, 1)

    s = Session(0)
    table = s.rope_table(_ffi.ROPE_GEMMA, D, base, position_divisor=divisor, max_positions=P + 8)
    cache = s.kv_cache(Hkv, D, P + 1)
    cache.append(pk, pv, P)
    dq, dk, dv, dqn, dkn = (torch.from_numpy(x).cuda() for x in (q, k, v, qn, kn))
    s.gemma_qk_prologue(table, dq, dk, 1, Hq, Hkv, D, dqn, dkn, eps, P, 1.0)
    out = torch.empty_like(dq)
    s.attention(dq, dk, dv, cache, KvAttentionConfig(1, Hq, Hkv, D, True, window), out)
    s.append(cache, dk, dv, 1)
    s.sync()
    assert_bitwise(dq.cpu().numpy(), rq, "prologue q")
    assert_bitwise(dk.cpu().numpy(), rk, "prologue k")
    err = rel_err(out.cpu().numpy(), want)
    print(f"[gemma] decode @32768 {name}: rel err {err:.2e}", flush=True)
    assert err <= DECODE_TOL
    assert_bitwise(cache.keys()[P * D:], ref_cache.keys()[P * D:], "appended key")
