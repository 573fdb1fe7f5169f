"""GPU parity of cached attention against the CPU oracle on identical seeded inputs.

Tolerances (metric: max|gpu - ref| / max|ref| over the output tensor):
  f32 decode (query_len == 1)         <= 1e-4
  f32 prefill precision (SIMT kernel) <= 1e-4
  bf16-MFMA prefill                   <= 1e-2
Shapes are the BASELINE configs' head geometry at contexts the oracle finishes
in seconds; full contexts are checked in test_gpu_scale.py.
"""
import numpy as np
import pytest

import oracle as o
from tests.helpers import layer_inputs, rel_err

pytestmark = pytest.mark.gpu

DECODE_TOL = 1e-4
F32_TOL = 1e-4
BF16_TOL = 1e-2


def run_both(gpu, config, layer, S, P, Hq, Hkv, D, window=0, causal=True, cap_extra=1):
    q, k, v, pk, pv = layer_inputs(config, layer, S, P, Hq, Hkv, D)
    cap = P + S + cap_extra
    ref_cache = o.KvCache(Hkv, D, cap)
    dev_cache = gpu.KvCache(Hkv, D, cap)
    if P:
        ref_cache.append(pk, pv, P)
        dev_cache.append(pk, pv, P)
    ref = o.sdpa_with_cache(q, k, v, ref_cache, S, Hq, Hkv, D, causal, window)
    cfg = gpu.KvAttentionConfig(S, Hq, Hkv, D, causal, window)
    got = gpu.scaled_dot_product_attention_with_cache(q, k, v, dev_cache, cfg)
    return got, ref, dev_cache, (q, k, v)


@pytest.mark.parametrize("name,P,Hq,Hkv,D,window", [
    ("cfg1 llama-1B @512", 512, 32, 8, 64, 0),
    ("cfg3b llama-3B @8192", 8192, 24, 8, 128, 0),
    ("cfg4 gemma-1B global @32768", 32768, 4, 1, 256, 0),
    ("cfg4 gemma-1B local W512 @32768", 32768, 4, 1, 256, 512),
    ("cfg5 gemma-4B global @16640", 16640, 8, 4, 256, 0),
    ("cfg5 gemma-4B local W1024", 16640, 8, 4, 256, 1024),
    ("first token", 0, 24, 8, 128, 0),
    ("window 1", 300, 8, 2, 64, 1),
    ("odd length", 1001, 12, 4, 128, 0),
    ("R=8", 2050, 32, 4, 64, 0),
    ("R=5", 777, 10, 2, 128, 0),
])
def test_decode_f32_parity(gpu, name, P, Hq, Hkv, D, window):
    print(f"[case] decode {name} P={P} Hq={Hq} Hkv={Hkv} D={D} W={window}", flush=True)
    got, ref, _, _ = run_both(gpu, 10, P % 97, 1, P, Hq, Hkv, D, window)
    assert rel_err(got, ref) <= DECODE_TOL


@pytest.mark.parametrize("D", [2, 6, 48, 96, 160])
def test_decode_generic_head_dims(gpu, D):
    got, ref, _, _ = run_both(gpu, 11, D, 1, 123, 6, 3, D)
    assert rel_err(got, ref) <= DECODE_TOL


@pytest.mark.parametrize("name,S,P,Hq,Hkv,D,window", [
    ("cfg2 llama-1B prefill", 512, 0, 32, 8, 64, 0),
    ("cfg3a llama-3B prefill", 512, 0, 24, 8, 128, 0),
    ("cfg4 gemma-1B prefill global", 300, 0, 4, 1, 256, 0),
    ("cfg4 gemma-1B prefill local W64", 300, 0, 4, 1, 256, 64),
    ("cfg5 gemma-4B chunk @4096", 128, 4096, 8, 4, 256, 0),
    ("cfg5 gemma-4B chunk local W1024", 128, 4096, 8, 4, 256, 1024),
    ("chunk with unaligned past", 45, 333, 24, 8, 128, 0),
    ("two tokens", 2, 5, 8, 2, 64, 0),
    ("33 tokens", 33, 0, 6, 2, 128, 0),
    ("R=8", 70, 10, 32, 4, 64, 0),
    ("R=1 MHA", 100, 3, 4, 4, 128, 0),
    # head_dim 128 with a window: rows whose first key tile lies wholly
    # outside their window have seen no key after the first tile
    ("llama-3B shape local W64", 300, 0, 24, 8, 128, 64),
    ("llama-3B shape chunk local W100", 96, 500, 24, 8, 128, 100),
])
def test_prefill_bf16_parity(gpu, name, S, P, Hq, Hkv, D, window):
    print(f"[case] prefill {name} S={S} P={P} Hq={Hq} Hkv={Hkv} D={D} W={window}", flush=True)
    got, ref, _, _ = run_both(gpu, 12, S + P, S, P, Hq, Hkv, D, window)
    assert rel_err(got, ref) <= BF16_TOL


@pytest.mark.parametrize("S,P,Hq,Hkv", [
    (1024, 0, 32, 8),  # Llama-3.2-1B heads (R = 4: two heads per workgroup)
    (333, 0, 16, 8),   # R = 2
    (700, 0, 24, 8),   # R = 3: one head, two query blocks per workgroup
    (129, 7, 8, 8),    # R = 1, a few cached keys, an odd tile count
    (2048, 0, 4, 1),   # pairs with key splits (128 paired workgroups)
    (1024, 0, 8, 2),   # pairs with key splits grouped by XCD
])
def test_prefill_wave_pairs(gpu, S, P, Hq, Hkv):
    """Head_dim-64 causal prompts run wave pairs (two waves take alternate
    key tiles of one query block and merge through LDS); every head grouping
    of the pair launcher against the oracle."""
    from spissa_amd.device import plan_attention

    D = 64
    plan = plan_attention(gpu.KvAttentionConfig(S, Hq, Hkv, D, True, 0), [P])
    print(f"[case] prefill wave pairs S={S} P={P} Hq={Hq} Hkv={Hkv} plan={plan['block_waves']}", flush=True)
    assert plan["block_waves"] == 2
    got, ref, _, _ = run_both(gpu, 31, S, S, P, Hq, Hkv, D)
    assert rel_err(got, ref) <= BF16_TOL


def test_prefill_non_causal(gpu):
    got, ref, _, _ = run_both(gpu, 13, 0, 64, 20, 8, 2, 128, 0, causal=False)
    assert rel_err(got, ref) <= BF16_TOL


def test_prefill_f32_precision_path(gpu):
    from spissa_amd import _ffi
    from spissa_amd.device import Session  # noqa: F401

    import ctypes

    lib = _ffi.load()
    h = ctypes.c_void_p()
    assert lib.spissa_default_session(ctypes.byref(h)) == 0
    assert lib.spissa_session_set_prefill_precision(h, _ffi.PREFILL_F32) == 0
    try:
        got, ref, _, _ = run_both(gpu, 14, 0, 200, 50, 24, 8, 128, 0)
        assert rel_err(got, ref) <= F32_TOL
    finally:
        lib.spissa_session_set_prefill_precision(h, _ffi.PREFILL_BF16)


def test_prefill_then_cache_append_then_decode_matches_full_recompute(gpu):
    # tiny.rs:1801-1898 pattern: prefill + decode steps == full-context recompute per step.
    Hq, Hkv, D, S0, steps = 8, 2, 64, 40, 5
    n = S0 + steps
    q, k, v, _, _ = layer_inputs(15, 0, n, 0, Hq, Hkv, D)
    full = o.sdpa_with_cache(q, k, v, None, n, Hq, Hkv, D)
    cache = gpu.KvCache(Hkv, D, n)
    qw, kw = Hq * D, Hkv * D
    out = gpu.scaled_dot_product_attention_with_cache(
        q[:S0 * qw].copy(), k[:S0 * kw].copy(), v[:S0 * kw].copy(), cache, gpu.KvAttentionConfig(S0, Hq, Hkv, D, True))
    cache.append(k[:S0 * kw].copy(), v[:S0 * kw].copy(), S0)
    assert rel_err(out, full[:S0 * qw]) <= BF16_TOL
    for t in range(S0, n):
        qs, ks, vs = q[t * qw:(t + 1) * qw].copy(), k[t * kw:(t + 1) * kw].copy(), v[t * kw:(t + 1) * kw].copy()
        got = gpu.scaled_dot_product_attention_with_cache(qs, ks, vs, cache, gpu.KvAttentionConfig(1, Hq, Hkv, D, True))
        cache.append(ks, vs, 1)
        assert rel_err(got, full[t * qw:(t + 1) * qw]) <= DECODE_TOL


def test_reference_kats_through_the_gpu(gpu):
    # rotary.rs:827-851 and ops.rs:537-554 through the drop-in entry points.
    f = lambda *x: np.array(x, dtype=np.float32)
    q_all, k_all, v_all = f(0.2, 0.7, -0.1, 0.4, 0.9, -0.3), f(0.5, -0.2, 0.1, 0.8, -0.4, 0.3), f(1.0, 0.0, -0.5, 2.0, 0.25, -1.0)
    full = o.scaled_dot_product_attention(q_all, k_all, v_all, 3, 1, 2, True)
    c = gpu.KvCache(1, 2, 3)
    c.append(k_all[:4].copy(), v_all[:4].copy(), 2)
    inc = gpu.scaled_dot_product_attention_with_cache(q_all[4:].copy(), k_all[4:].copy(), v_all[4:].copy(), c,
                                                      gpu.KvAttentionConfig(1, 1, 1, 2, True))
    np.testing.assert_allclose(inc, full[4:], atol=1e-6, rtol=0)
    q = f(1.0, 0.0, 0.0, 1.0)
    out = gpu.scaled_dot_product_attention(q, q.copy(), f(10.0, 0.0, 0.0, 20.0), 2, 1, 2, True)
    np.testing.assert_allclose(out[:2], [10.0, 0.0], atol=1e-6)
    assert 3.0 < out[2] < 3.4 and 13.0 < out[3] < 13.7


@pytest.mark.parametrize("D,Hq,Hkv", [(64, 8, 2), (128, 6, 2), (256, 4, 1)])
def test_prefill_reference_rises_across_tiles(gpu, D, Hq, Hkv):
    """Scores that jump by about 140 (log2 units) after the first 64 keys: the
    exponent reference taken from the first key tile is far too low for the
    rest, so the kernel must raise it (lazily from the probability sums at
    head_dim 128, from the next tile's row maxima otherwise); without the
    raise the later probabilities would overflow to inf (2^140). Compared
    with the oracle on the same inputs."""
    S = 320
    print(f"[case] prefill reference rise D={D} Hq={Hq} Hkv={Hkv} S={S}", flush=True)
    q, k, v, _, _ = layer_inputs(17, D, S, 0, Hq, Hkv, D)
    # a common component of every query row along dim 0, and keys 0..63
    # pointing against it: their scores sit ~140 log2 units below the rest
    amp = float(np.sqrt(140.0 / 1.4426950408889634 * np.sqrt(D)))
    q = q.reshape(S, Hq, D)
    q[:, :, 0] += amp
    k = k.reshape(S, Hkv, D)
    k[:64, :, 0] -= amp
    k[64:, :, 0] = 0.0  # the later keys' scores stay moderate (no amp x k term)
    q, k = q.ravel().copy(), k.ravel().copy()
    ref = o.sdpa_with_cache(q, k, v, None, S, Hq, Hkv, D, True, 0)
    got = gpu.scaled_dot_product_attention_with_cache(q, k, v, None, gpu.KvAttentionConfig(S, Hq, Hkv, D, True))
    assert np.all(np.isfinite(got))
    # Rows 64.. see the later keys, whose scores are moderate, so bf16 scores
    # are accurate there. (Rows 0-63 see only the shifted keys, whose large
    # raw scores carry bf16 rounding errors of several units; they never need
    # a raise.)
    lo = 64 * Hq * D
    assert rel_err(got[lo:], ref[lo:]) <= BF16_TOL


@pytest.mark.parametrize("D,Hq,Hkv", [(64, 8, 2), (128, 6, 2), (256, 4, 1)])
def test_prefill_rows_first_seeing_keys_far_below_zero(gpu, D, Hq, Hkv):
    """Windowed causal prefill whose scores all sit about 130 log2 units below
    zero: the rows whose window starts past a workgroup's first key tile have
    accumulated nothing (m = -inf) when their first visible keys arrive, and
    their rescale factor must be 0, not 2^130 (0 x inf = NaN). The common
    score offset comes from dim 0 set to +-amp in q and k, exact in bf16, so
    the bf16 scores stay accurate relative to each other."""
    S, W = 320, 100
    amp = 40.0 if D <= 128 else 48.0  # amp^2 / sqrt(D) x log2(e) > 128; exact in bf16
    print(f"[case] prefill far-negative scores D={D} Hq={Hq} Hkv={Hkv} S={S} W={W}", flush=True)
    q, k, v, _, _ = layer_inputs(29, D, S, 0, Hq, Hkv, D)
    q = q.reshape(S, Hq, D)
    k = k.reshape(S, Hkv, D)
    q[:, :, 0] = amp
    k[:, :, 0] = -amp  # every score gets -amp^2 / sqrt(D)
    q, k = q.ravel().copy(), k.ravel().copy()
    ref = o.sdpa_with_cache(q, k, v, None, S, Hq, Hkv, D, True, W)
    got = gpu.scaled_dot_product_attention_with_cache(q, k, v, None, gpu.KvAttentionConfig(S, Hq, Hkv, D, True, W))
    assert np.all(np.isfinite(got))
    assert rel_err(got, ref) <= BF16_TOL


def test_invalid_softmax_denominator_is_reported(gpu):
    P, Hq, Hkv, D = 64, 8, 2, 128
    q, k, v, pk, pv = layer_inputs(16, 0, 1, P, Hq, Hkv, D)
    cache = gpu.KvCache(Hkv, D, P + 1)
    cache.append(pk, pv, P)
    q[5] = np.nan
    with pytest.raises(gpu.InvalidTensorDataError):
        gpu.scaled_dot_product_attention_with_cache(q, k, v, cache, gpu.KvAttentionConfig(1, Hq, Hkv, D, True))
    # The session recovers: a valid call afterwards succeeds.
    q[5] = 0.0
    gpu.scaled_dot_product_attention_with_cache(q, k, v, cache, gpu.KvAttentionConfig(1, Hq, Hkv, D, True))


def test_split_prefill_ignores_stale_partials_of_empty_splits(gpu):
    """A causal prefill with key splits: the early query blocks' upper splits
    see no key and write no partial O. A non-causal call of the same size
    first fills the same workspace with NaN partials. The combine must skip
    the empty splits rather than scale the stale NaNs by zero."""
    S, Hq, Hkv, D = 1024, 4, 1, 256  # 32 workgroups: 7 key splits, most empty for early blocks
    q, k, v, _, _ = layer_inputs(17, 0, S, 0, Hq, Hkv, D)
    with pytest.raises(gpu.InvalidTensorDataError):
        gpu.scaled_dot_product_attention_with_cache(np.full_like(q, np.nan), k, v, None,
                                                    gpu.KvAttentionConfig(S, Hq, Hkv, D, False))
    got = gpu.scaled_dot_product_attention_with_cache(q, k, v, None, gpu.KvAttentionConfig(S, Hq, Hkv, D, True))
    ref = o.sdpa_with_cache(q, k, v, None, S, Hq, Hkv, D, True, 0)
    assert np.all(np.isfinite(got))
    err = rel_err(got, ref)
    print(f"[prefill] stale-workspace split case: rel err {err:.2e}", flush=True)
    assert err <= BF16_TOL


def test_batched_decode_matches_per_sequence_oracle(gpu):
    import torch

    from spissa_amd.device import Session

    B, Hq, Hkv, D = 16, 24, 8, 128
    lens = [100 + 37 * b for b in range(B)]
    s = Session(0)
    caches, refs, qs, ks, vs = [], [], [], [], []
    for b in range(B):
        q, k, v, pk, pv = layer_inputs(17, 0, 1, lens[b], Hq, Hkv, D, sequence=b)
        c = s.kv_cache(Hkv, D, lens[b] + 1)
        c.append(pk, pv, lens[b])
        rc = o.KvCache(Hkv, D, lens[b] + 1)
        rc.append(pk, pv, lens[b])
        refs.append(o.sdpa_with_cache(q, k, v, rc, 1, Hq, Hkv, D))
        caches.append(c)
        qs.append(q), ks.append(k), vs.append(v)
    dq = torch.from_numpy(np.concatenate(qs)).cuda()
    dk = torch.from_numpy(np.concatenate(ks)).cuda()
    dv = torch.from_numpy(np.concatenate(vs)).cuda()
    out = torch.empty_like(dq)
    s.attention_decode_batch(dq, dk, dv, caches, gpu.KvAttentionConfig(1, Hq, Hkv, D, True), out)
    s.sync()
    got = out.cpu().numpy().reshape(B, -1)
    for b in range(B):
        assert rel_err(got[b], refs[b]) <= DECODE_TOL, b


@pytest.mark.parametrize("kind,Hq,Hkv,D,P,window,base,div", [
    ("llama-3B", 24, 8, 128, 2000, 0, 500000.0, 1.0),
    ("llama-1B", 32, 8, 64, 511, 0, 500000.0, 1.0),
    ("gemma-1B global", 4, 1, 256, 700, 0, 1e6, 8.0),
    ("gemma-4B local", 8, 4, 256, 1500, 1024, 10000.0, 1.0),
    ("first token", 24, 8, 128, 0, 0, 500000.0, 1.0),
])
def test_fused_decode_step_matches_rope_sdpa_append(gpu, kind, Hq, Hkv, D, P, window, base, div):
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session

    print(f"[case] fused decode {kind} P={P}", flush=True)
    steps = 3
    s = Session(0)
    gemma = kind.startswith("gemma")
    table = s.rope_table(_ffi.ROPE_GEMMA if gemma else _ffi.ROPE_LLAMA, D, base, div, max_positions=P + steps + 8)
    cache = s.kv_cache(Hkv, D, P + steps)
    ref = o.KvCache(Hkv, D, P + steps)
    _, _, _, pk, pv = layer_inputs(20, 1, 1, P, Hq, Hkv, D)
    if P:
        cache.append(pk, pv, P)
        ref.append(pk, pv, P)
    cfg = gpu.KvAttentionConfig(1, Hq, Hkv, D, True, window)
    for t in range(steps):
        q, k, v, _, _ = layer_inputs(21, t, 1, 0, Hq, Hkv, D)
        rq, rk = q.copy(), k.copy()
        if gemma:
            o.apply_gemma_rotary_inplace(rq, rk, Hq, Hkv, 1, D, D, base, P + t, div)
        else:
            o.apply_llama_rotary_inplace(rq, rk, Hq, Hkv, 1, D, D, base, P + t)
        want = o.sdpa_with_cache(rq, rk, v, ref, 1, Hq, Hkv, D, True, window)
        ref.append(rk, v, 1)
        dq, dk, dv = (torch.from_numpy(x).cuda() for x in (q, k, v))
        out = torch.empty_like(dq)
        s.decode_step(table, dq, dk, dv, [cache], cfg, out)
        s.sync()
        assert rel_err(out.cpu().numpy(), want) <= DECODE_TOL
        assert cache.len() == P + t + 1
        assert np.array_equal(dq.cpu().numpy(), q) and np.array_equal(dk.cpu().numpy(), k), "inputs are read-only"
    from tests.helpers import assert_bitwise
    assert_bitwise(cache.keys(), ref.keys(), "keys after fused appends")
    assert_bitwise(cache.values(), ref.values(), "values after fused appends")
    with pytest.raises(gpu.ShapeError):  # full cache: validated before launching, nothing mutated
        s.decode_step(table, dq, dk, dv, [cache], cfg, out)
    assert cache.len() == P + steps


def test_fused_decode_batch_after_prefill_keeps_shadow_consistent(gpu):
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session

    B, Hq, Hkv, D, S0 = 4, 8, 2, 128, 300
    s = Session(0)
    table = s.rope_table(_ffi.ROPE_LLAMA, D, 500000.0, max_positions=1024)
    caches, refs = [], []
    for b in range(B):
        q, k, v, _, _ = layer_inputs(22, 0, S0 + 7 * b, 0, Hq, Hkv, D, sequence=b)
        c, rc = s.kv_cache(Hkv, D, 512), o.KvCache(Hkv, D, 512)
        n = S0 + 7 * b
        dq, dk, dv = (torch.from_numpy(x).cuda() for x in (q, k, v))
        dout = torch.empty_like(dq)
        s.attention(dq, dk, dv, c, gpu.KvAttentionConfig(n, Hq, Hkv, D, True), dout)  # builds no shadow (P=0)
        c.append(k, v, n)
        rc.append(k, v, n)
        caches.append(c), refs.append(rc)
    # a chunked prefill on cache 0 creates its bf16 shadow
    q, k, v, _, _ = layer_inputs(23, 0, 16, 0, Hq, Hkv, D)
    got = gpu.scaled_dot_product_attention_with_cache(q, k, v, caches[0], gpu.KvAttentionConfig(16, Hq, Hkv, D, True))
    assert rel_err(got, o.sdpa_with_cache(q, k, v, refs[0], 16, Hq, Hkv, D)) <= BF16_TOL
    cfg = gpu.KvAttentionConfig(1, Hq, Hkv, D, True)
    # 12 steps move cache 0 from 316 to 328 tokens, so the next chunk reads the
    # shadow rows written by the fused appends (below the 8-aligned restaging tail).
    for t in range(12):
        qs, ks, vs, wants = [], [], [], []
        for b in range(B):
            q, k, v, _, _ = layer_inputs(24, t, 1, 0, Hq, Hkv, D, sequence=b)
            rq, rk = q.copy(), k.copy()
            o.apply_llama_rotary_inplace(rq, rk, Hq, Hkv, 1, D, D, 500000.0, refs[b].len())
            wants.append(o.sdpa_with_cache(rq, rk, v, refs[b], 1, Hq, Hkv, D))
            refs[b].append(rk, v, 1)
            qs.append(q), ks.append(k), vs.append(v)
        dq, dk, dv = (torch.from_numpy(np.concatenate(x)).cuda() for x in (qs, ks, vs))
        out = torch.empty_like(dq)
        s.decode_step(table, dq, dk, dv, caches, cfg, out)
        s.sync()
        got = out.cpu().numpy().reshape(B, -1)
        for b in range(B):
            assert rel_err(got[b], wants[b]) <= DECODE_TOL
    # the shadow of cache 0 followed the fused appends: another chunk agrees with the oracle
    q, k, v, _, _ = layer_inputs(25, 0, 9, 0, Hq, Hkv, D)
    got = gpu.scaled_dot_product_attention_with_cache(q, k, v, caches[0], gpu.KvAttentionConfig(9, Hq, Hkv, D, True))
    assert rel_err(got, o.sdpa_with_cache(q, k, v, refs[0], 9, Hq, Hkv, D)) <= BF16_TOL


@pytest.mark.parametrize("S,P,Hq,Hkv,D,W", [(256, 4100, 32, 8, 64, 512), (128, 3000, 16, 4, 128, 1024)])
def test_prefill_windowed_non_causal_with_key_splits(gpu, S, P, Hq, Hkv, D, W):
    """A windowed non-causal chunk over a long cache takes key splits, and a
    block's range then runs from its first query's window to the last key:
    every split range must be covered (the oracle applies the same window)."""
    print(f"[case] prefill non-causal window S={S} P={P} Hq={Hq} Hkv={Hkv} D={D} W={W}", flush=True)
    got, ref, _, _ = run_both(gpu, 26, S, S, P, Hq, Hkv, D, W, causal=False)
    assert rel_err(got, ref) <= BF16_TOL


def test_decode_step_rejects_a_cache_listed_twice(gpu):
    import torch

    from spissa_amd.device import Session

    Hq, Hkv, D = 8, 2, 64
    s = Session(0)
    c0, c1 = s.kv_cache(Hkv, D, 8), s.kv_cache(Hkv, D, 8)
    q = torch.zeros(3, Hq, D, device="cuda")
    k = torch.zeros(3, Hkv, D, device="cuda")
    out = torch.empty_like(q)
    with pytest.raises(gpu.ArgumentError):
        s.decode_step(None, q, k, k.clone(), [c0, c1, c0], gpu.KvAttentionConfig(1, Hq, Hkv, D, True), out)
    assert c0.len() == 0 and c1.len() == 0  # nothing appended
    s.decode_step(None, q[:2], k[:2], k[:2].clone(), [c0, c1], gpu.KvAttentionConfig(1, Hq, Hkv, D, True), out[:2])
    s.sync()
    assert c0.len() == 1 and c1.len() == 1


def test_workspace_growth_under_graph_capture_is_a_clear_error(gpu):
    """A call whose workspace would grow while its stream is captured returns
    ERR_ARGUMENT with a message instead of a device error; the same call
    after an uncaptured warm-up captures and replays."""
    import torch

    from spissa_amd.device import Session

    S, Hq, Hkv, D = 64, 8, 2, 128
    st = torch.cuda.Stream()
    s = Session(0, stream=st)
    q = torch.randn(S, Hq, D, device="cuda")
    k = torch.randn(S, Hkv, D, device="cuda")
    v = torch.randn(S, Hkv, D, device="cuda")
    out = torch.empty_like(q)
    cfg = gpu.KvAttentionConfig(S, Hq, Hkv, D, True)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    raised = None
    with torch.cuda.graph(g, stream=st):
        try:
            s.attention(q, k, v, None, cfg, out)
        except gpu.ArgumentError as e:
            raised = str(e)
    assert raised is not None and "captured" in raised, raised
    s.attention(q, k, v, None, cfg, out)  # warm-up: the workspace grows here
    s.sync()
    want = out.clone()
    out.zero_()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=st):
        s.attention(q, k, v, None, cfg, out)
    for _ in range(3):
        out.zero_()
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
