"""Pins the CPU oracle beyond the reference's tiny KATs.

Independent float64 brute force (numpy, written from the mathematics, not
from the oracle's loops), closed forms and invariants at realistic head
dimensions. Chosen so a plausible restatement mistake fails at least one of
them: a wrong kv-head mapping or GQA grouping (GQA == replicated MHA, f64 brute
force), a wrong causal or window bound (brute force with masks, W >= key_len
identity), a dropped scale (closed form), a swapped rotate-half sign or pair
index (f64 rotation, pos-0 identity, norm preservation).
"""
import ctypes
import ctypes.util
import math

import numpy as np
import pytest

import oracle as o
from spissa_amd.synth import normal_f32, seed_for
from tests.helpers import assert_bitwise, rel_err


def _libm():
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.powf.restype = ctypes.c_float
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    return libm


def brute_sdpa_f64(q, k_all, v_all, S, P, Hq, Hkv, D, causal=True, window=0):
    """Float64 attention: q [S,Hq,D], k_all/v_all [P+S,Hkv,D] (cache rows then current rows)."""
    q = q.reshape(S, Hq, D).astype(np.float64)
    K = k_all.reshape(P + S, Hkv, D).astype(np.float64)
    V = v_all.reshape(P + S, Hkv, D).astype(np.float64)
    out = np.zeros((S, Hq, D))
    r = Hq // Hkv
    keys = np.arange(P + S)
    for i in range(S):
        qa = P + i
        vis = np.ones(P + S, dtype=bool)
        if causal:
            vis &= keys <= qa
        if window:
            vis &= keys + window > qa
        for h in range(Hq):
            g = h // r
            s = K[vis, g, :] @ q[i, h] / math.sqrt(D)
            p = np.exp(s - s.max())
            p /= p.sum()
            out[i, h] = p @ V[vis, g, :]
    return out.ravel()


def cache_with(k, v, Hkv, D, cap):
    c = o.KvCache(Hkv, D, cap)
    if k.size:
        c.append(k, v, k.size // (Hkv * D))
    return c


@pytest.mark.parametrize("S,P,Hq,Hkv,D,window", [
    (1, 37, 8, 2, 64, 0), (1, 100, 6, 2, 128, 16), (5, 11, 4, 1, 32, 0), (7, 0, 4, 4, 16, 3),
    (3, 9, 6, 3, 8, 0)])
def test_sdpa_matches_float64_brute_force(S, P, Hq, Hkv, D, window):
    q = normal_f32(11, S * Hq * D)
    ka = normal_f32(12, (P + S) * Hkv * D)
    va = normal_f32(13, (P + S) * Hkv * D)
    w = Hkv * D
    c = cache_with(ka[:P * w].copy(), va[:P * w].copy(), Hkv, D, P + S + 1)
    got = o.sdpa_with_cache(q, ka[P * w:].copy(), va[P * w:].copy(), c, S, Hq, Hkv, D, True, window)
    ref = brute_sdpa_f64(q, ka, va, S, P, Hq, Hkv, D, True, window)
    assert rel_err(got, ref) < 2e-6


def test_gqa_equals_mha_with_replicated_kv():
    S, P, Hq, Hkv, D = 3, 20, 8, 2, 16
    r = Hq // Hkv
    q = normal_f32(21, S * Hq * D)
    ka, va = normal_f32(22, (P + S) * Hkv * D), normal_f32(23, (P + S) * Hkv * D)
    rep = lambda a: np.repeat(a.reshape(-1, Hkv, D), r, axis=1).ravel().copy()
    w = Hkv * D
    gqa = o.sdpa_with_cache(q, ka[P * w:].copy(), va[P * w:].copy(),
                            cache_with(ka[:P * w].copy(), va[:P * w].copy(), Hkv, D, 64), S, Hq, Hkv, D)
    kr, vr = rep(ka), rep(va)
    wr = Hq * D
    mha = o.sdpa_with_cache(q, kr[P * wr:].copy(), vr[P * wr:].copy(),
                            cache_with(kr[:P * wr].copy(), vr[:P * wr].copy(), Hq, D, 64), S, Hq, Hq, D)
    assert_bitwise(gqa, mha, "GQA vs replicated MHA")


def test_chunked_prefill_equals_one_shot_rows():
    S, Hq, Hkv, D = 24, 4, 2, 16
    q = normal_f32(31, S * Hq * D)
    k, v = normal_f32(32, S * Hkv * D), normal_f32(33, S * Hkv * D)
    one = o.sdpa_with_cache(q, k, v, None, S, Hq, Hkv, D)
    c = o.KvCache(Hkv, D, S)
    parts = []
    for a, b in ((0, 7), (7, 8), (8, 24)):
        qs, ks, vs = (x[a * n * D:b * n * D].copy() for x, n in ((q, Hq), (k, Hkv), (v, Hkv)))
        parts.append(o.sdpa_with_cache(qs, ks, vs, c, b - a, Hq, Hkv, D))
        c.append(ks, vs, b - a)
    assert_bitwise(np.concatenate(parts), one, "chunked vs one-shot")


def test_window_wider_than_context_is_the_reference():
    S, P, Hq, Hkv, D = 4, 30, 4, 1, 16
    q = normal_f32(41, S * Hq * D)
    ka, va = normal_f32(42, (P + S) * Hkv * D), normal_f32(43, (P + S) * Hkv * D)
    w = Hkv * D
    args = (q, ka[P * w:].copy(), va[P * w:].copy())
    c = cache_with(ka[:P * w].copy(), va[:P * w].copy(), Hkv, D, 64)
    base = o.sdpa_with_cache(*args, c, S, Hq, Hkv, D, True, 0)
    wide = o.sdpa_with_cache(*args, c, S, Hq, Hkv, D, True, P + S)
    assert_bitwise(wide, base, "window >= key_len")
    narrow = o.sdpa_with_cache(*args, c, S, Hq, Hkv, D, True, 5)
    assert rel_err(narrow, base) > 1e-3


def test_zero_query_gives_mean_of_visible_values():
    S, P, Hq, Hkv, D, W = 3, 10, 2, 1, 8, 6
    q = np.zeros(S * Hq * D, dtype=np.float32)
    ka, va = normal_f32(51, (P + S) * Hkv * D), normal_f32(52, (P + S) * Hkv * D)
    w = Hkv * D
    got = o.sdpa_with_cache(q, ka[P * w:].copy(), va[P * w:].copy(),
                            cache_with(ka[:P * w].copy(), va[:P * w].copy(), Hkv, D, 32), S, Hq, Hkv, D, True, W)
    V = va.reshape(P + S, D).astype(np.float64)
    for i in range(S):
        qa = P + i
        mean = V[qa - W + 1:qa + 1].mean(axis=0)
        for h in range(Hq):
            np.testing.assert_allclose(got.reshape(S, Hq, D)[i, h], mean, rtol=0, atol=2e-6)


def test_one_hot_key_selects_its_value_row():
    # A query aligned with one key (score 60 vs 0) puts ~all weight on that key's value row.
    D, P = 16, 9
    K = np.zeros((P + 1, 1, D), dtype=np.float32)
    K[4, 0, 0] = 1.0
    V = normal_f32(61, (P + 1) * D).reshape(P + 1, 1, D)
    q = np.zeros(D, dtype=np.float32)
    q[0] = 240.0  # score 240/sqrt(16) = 60 for key 4, 0 elsewhere
    c = cache_with(K[:P].ravel().copy(), V[:P].ravel().copy(), 1, D, 16)
    got = o.sdpa_with_cache(q, K[P].ravel().copy(), V[P].ravel().copy(), c, 1, 1, 1, D)
    np.testing.assert_allclose(got, V[4, 0], rtol=0, atol=1e-6)


@pytest.mark.parametrize("kind", ["llama", "gemma", "neox"])
def test_rope_matches_float64_rotation_of_the_f32_angle(kind):
    S, H, D, off = 5, 3, 64, 8190
    base, div = (500000.0, 8.0) if kind != "neox" else (10000.0, 1.0)
    x = normal_f32(71, S * H * D)
    q, k = x.copy(), x.copy()
    if kind == "llama":
        o.apply_llama_rotary_inplace(q, k, H, H, S, D, D, base, off)
    elif kind == "gemma":
        o.apply_gemma_rotary_inplace(q, k, H, H, S, D, D, base, off, div)
    else:
        o.apply_gpt_neox_rotary_inplace(q, k, S, H, D, D, base, off)
    half = D // 2
    X = x.reshape(S, H, D).astype(np.float64)
    ref = X.copy()
    powf = _libm().powf  # Rust's f32::powf is glibc powf on x86_64-linux-gnu
    for s in range(S):
        for p in range(half):
            inv = np.float32(1.0) / np.float32(powf(base, float(np.float32(2 * p) / np.float32(D))))
            pos = np.float32(off + s) / np.float32(div) if kind == "gemma" else np.float32(off + s)
            ang = float(np.float32(pos * inv))
            c, sn = math.cos(ang), math.sin(ang)
            a, b = X[s, :, p], X[s, :, p + half]
            ref[s, :, p] = a * c - b * sn
            ref[s, :, p + half] = b * c + a * sn
    assert rel_err(q, ref.ravel()) < 1e-6
    assert_bitwise(q, k, "q and k rotate identically")


def test_rope_at_position_zero_is_identity_and_preserves_pair_norms():
    S, H, D = 4, 2, 32
    x = normal_f32(81, S * H * D)
    q, k = x[:H * D].copy(), x[:H * D].copy()
    o.apply_llama_rotary_inplace(q, k, H, H, 1, D, D, 500000.0, 0)
    assert_bitwise(q, x[:H * D], "pos 0 identity")
    q, k = x.copy(), x.copy()
    o.apply_llama_rotary_inplace(q, k, H, H, S, D, D, 500000.0, 1234)
    n0 = x.reshape(-1, 2, D // 2).astype(np.float64)
    n1 = q.reshape(-1, 2, D // 2).astype(np.float64)
    np.testing.assert_allclose((n1 ** 2).sum(axis=1), (n0 ** 2).sum(axis=1), rtol=1e-5)


def test_rms_norm_matches_float64():
    rows, cols = 33, 256
    x, w = normal_f32(91, rows * cols), normal_f32(92, cols, 1.0, 0.1)
    got = o.rms_norm(x, w, rows, cols, 1e-6)
    X = x.reshape(rows, cols).astype(np.float64)
    ref = X / np.sqrt((X ** 2).mean(axis=1, keepdims=True) + 1e-6) * w.astype(np.float64)
    assert rel_err(got, ref.ravel()) < 1e-6


def test_gemma_prologue_is_norm_then_rope_then_prescale():
    S, Hq, Hkv, D = 3, 4, 2, 32
    q, k = normal_f32(101, S * Hq * D), normal_f32(102, S * Hkv * D)
    qn, kn = normal_f32(103, D, 1.0, 0.1), normal_f32(104, D, 1.0, 0.1)
    qa, ka = q.copy(), k.copy()
    o.gemma_qk_prologue(qa, ka, S, Hq, Hkv, D, qn, kn, 1e-6, 1e6, 8.0, 17, 64.0)
    qb = o.rms_norm(q, qn, S * Hq, D, 1e-6)
    kb = o.rms_norm(k, kn, S * Hkv, D, 1e-6)
    o.apply_gemma_rotary_inplace(qb, kb, Hq, Hkv, S, D, D, 1e6, 17, 8.0)
    pre = np.float32(1.0) / np.sqrt(np.float32(64.0)) * np.sqrt(np.float32(D))
    assert_bitwise(ka, kb, "k")
    assert_bitwise(qa, qb * np.float32(pre), "q")


def test_softmax_denominator_error_on_non_finite_scores():
    q = np.array([np.nan, 0.0], dtype=np.float32)
    k = np.array([1.0, 0.0], dtype=np.float32)
    with pytest.raises(o.OracleError) as e:
        o.sdpa_with_cache(q, k, k.copy(), None, 1, 1, 1, 2)
    assert e.value.kind == "InvalidTensorData"


def test_glibc_sincosf_agrees_with_sinf_and_cosf_on_rope_angles():
    """Rust/LLVM may fuse x.cos() and x.sin() into one sincosf call; glibc's
    sincosf must then give the same bits as separate sinf and cosf."""
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.sinf.restype = libm.cosf.restype = ctypes.c_float
    libm.sinf.argtypes = libm.cosf.argtypes = [ctypes.c_float]
    libm.sincosf.restype = None
    libm.sincosf.argtypes = [ctypes.c_float, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]
    rng = np.random.default_rng(5)
    pos = rng.integers(0, 40000, 3000)
    pair = rng.integers(0, 128, 3000)
    s, c = ctypes.c_float(), ctypes.c_float()
    for p, i in zip(pos, pair):
        ang = np.float32(np.float32(p) * np.float32(0.9 ** float(i)))
        libm.sincosf(float(ang), ctypes.byref(s), ctypes.byref(c))
        assert s.value == libm.sinf(float(ang)) and c.value == libm.cosf(float(ang))


def test_seeded_inputs_are_reproducible():
    a = normal_f32(seed_for(3, 5, 0, "k", 2), 1000)
    b = normal_f32(seed_for(3, 5, 0, "k", 2), 1000)
    assert_bitwise(a, b, "same seed")
    assert abs(a.mean()) < 0.15 and 0.85 < a.std() < 1.15
