"""The attention sublayer on the device (spissa_attention_sublayer_device)
against the reference's own sequence restated on the CPU oracle
(models/gemma/generate.rs:178-312; models/llama/generate.rs:200-450):

    input rms_norm -> q/k/v projections -> QK-norm (Gemma) -> RoPE at the
    cache's next positions -> q prescale -> attention over cache + current rows
    -> append -> o projection -> post-attention rms_norm (Gemma)

Tolerances are those of the parts: 1e-4 of max |out| where the attention is
the f32 decode path, 1e-2 where it is the bf16-MFMA prefill; the appended
cache rows within 1e-4 (they come out of the f32 projections).
"""
import zlib

import numpy as np
import pytest

import oracle as o
from spissa_amd.linear import DTYPE_BF16
from spissa_amd.synth import normal_f32, seed_for
from tests.helpers import rel_err

pytestmark = pytest.mark.gpu


def seed(tag: str, n: int) -> int:
    return seed_for(97, n, 0, "q", zlib.crc32(tag.encode()))


def bf16_bits(x):
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


class Case:
    def __init__(self, name, kind, hidden, Hq, Hkv, D, P, S, base, divisor=1.0, window=0, qpas=None,
                 use_cache=True):
        self.__dict__.update(locals())
        del self.__dict__["self"]
        self.gemma = kind == "gemma"
        r = lambda tag, n, mean=0.0, std=1.0: normal_f32(seed(f"{name}.{tag}", n), n, mean, std)
        self.x = r("x", S * hidden)
        self.w = {t: bf16_bits(r(t, o_ * i_, 0.0, 0.02)) for t, (o_, i_) in
                  {"q": (Hq * D, hidden), "k": (Hkv * D, hidden), "v": (Hkv * D, hidden),
                   "o": (hidden, Hq * D)}.items()}
        self.in_norm = r("in_norm", hidden, 1.0, 0.1)
        self.q_norm = r("q_norm", D, 1.0, 0.1) if self.gemma else None
        self.k_norm = r("k_norm", D, 1.0, 0.1) if self.gemma else None
        self.post_norm = r("post_norm", hidden, 1.0, 0.1) if self.gemma else None
        self.past_k = r("past_k", P * Hkv * D)
        self.past_v = r("past_v", P * Hkv * D)
        self.eps = 1e-6
        qp = qpas if qpas is not None else D
        self.q_prescale = float(np.float32(1.0) / np.sqrt(np.float32(qp)) * np.sqrt(np.float32(D))) \
            if self.gemma else 1.0


CASES = [
    Case("llama3b_decode_p300", "llama", 3072, 24, 8, 128, 300, 1, 500000.0),
    Case("gemma1b_local_decode_p600_w512_qpas224", "gemma", 1152, 4, 1, 256, 600, 1, 10000.0, window=512,
         qpas=224),
    Case("gemma4b_global_chunk_s16_p100", "gemma", 2560, 8, 4, 256, 100, 16, 1000000.0, divisor=8.0),
    Case("llama1b_prefill_s64_nocache", "llama", 2048, 32, 8, 64, 0, 64, 500000.0, use_cache=False),
]


def run_oracle(c: Case):
    S, H, Hq, Hkv, D = c.S, c.hidden, c.Hq, c.Hkv, c.D
    xn = o.rms_norm(c.x, c.in_norm, S, H, c.eps)
    q = o.linear(xn, c.w["q"], o.DTYPE_BF16, None, S, H, Hq * D)
    k = o.linear(xn, c.w["k"], o.DTYPE_BF16, None, S, H, Hkv * D)
    v = o.linear(xn, c.w["v"], o.DTYPE_BF16, None, S, H, Hkv * D)
    if c.gemma:
        qpas = float(c.qpas if c.qpas is not None else D)
        o.gemma_qk_prologue(q, k, S, Hq, Hkv, D, c.q_norm, c.k_norm, c.eps, c.base, c.divisor, c.P, qpas)
    else:
        o.apply_llama_rotary_inplace(q, k, Hq, Hkv, S, D, D, c.base, c.P)
    cache = None
    if c.use_cache:
        cache = o.KvCache(Hkv, D, c.P + S)
        if c.P:
            cache.append(c.past_k.copy(), c.past_v.copy(), c.P)
    att = o.sdpa_with_cache(q, k, v, cache, S, Hq, Hkv, D, True, c.window)
    if cache is not None:
        cache.append(k, v, S)
    y = o.linear(att, c.w["o"], o.DTYPE_BF16, None, S, Hq * D, H)
    if c.gemma:
        y = o.rms_norm(y, c.post_norm, S, H, c.eps)
    return y, cache


@pytest.mark.parametrize("case", CASES, ids=lambda c: c.name)
def test_sublayer_matches_oracle_sequence(gpu, case):
    import torch

    from spissa_amd.device import AttentionLayer, Session

    c = case
    st = torch.cuda.Stream()
    s = Session(0, stream=st)
    W = {t: s.linear_weight(c.w[t], DTYPE_BF16, *shape) for t, shape in
         {"q": (c.Hq * c.D, c.hidden), "k": (c.Hkv * c.D, c.hidden), "v": (c.Hkv * c.D, c.hidden),
          "o": (c.hidden, c.Hq * c.D)}.items()}
    dev = lambda a: None if a is None else torch.from_numpy(a).cuda()
    kind = 1 if c.gemma else 0
    table = s.rope_table(kind, c.D, c.base, c.divisor, None, max_positions=c.P + c.S)
    layer = AttentionLayer(c.hidden, c.Hq, c.Hkv, c.D, W["q"], W["k"], W["v"], W["o"], dev(c.in_norm),
                           dev(c.q_norm), dev(c.k_norm), dev(c.post_norm), c.eps, table, c.q_prescale, True,
                           c.window)
    cache = None
    if c.use_cache:
        cache = s.kv_cache(c.Hkv, c.D, c.P + c.S)
        if c.P:
            cache.append(c.past_k.copy(), c.past_v.copy(), c.P)
    with torch.cuda.stream(st):
        x = dev(c.x)
        out = torch.empty(c.S * c.hidden, device="cuda")
        s.attention_sublayer(layer, x, c.S, cache, out)
    s.sync()
    ref, ref_cache = run_oracle(c)
    tol = 1e-4 if c.S == 1 else 1e-2
    err = rel_err(out.cpu().numpy(), ref)
    print(f"[sublayer] {c.name}: out rel err {err:.2e}", flush=True)
    assert err <= tol
    if cache is not None:
        assert cache.len() == c.P + c.S
        w = c.Hkv * c.D
        ek = rel_err(cache.keys()[c.P * w:], ref_cache.keys()[c.P * w:])
        ev = rel_err(cache.values()[c.P * w:], ref_cache.values()[c.P * w:])
        print(f"[sublayer] {c.name}: appended k {ek:.2e}, v {ev:.2e}", flush=True)
        assert ek <= 1e-4 and ev <= 1e-4
        assert np.array_equal(cache.keys()[:c.P * w], c.past_k)  # the past rows are untouched


def test_sublayer_errors_leave_the_cache_alone(gpu):
    import torch

    import spissa_amd as sa
    from spissa_amd.device import AttentionLayer, Session

    c = CASES[0]
    s = Session(0)
    W = {t: s.linear_weight(c.w[t], DTYPE_BF16, *shape) for t, shape in
         {"q": (c.Hq * c.D, c.hidden), "k": (c.Hkv * c.D, c.hidden), "v": (c.Hkv * c.D, c.hidden),
          "o": (c.hidden, c.Hq * c.D)}.items()}
    table = s.rope_table(0, c.D, c.base, 1.0, None, max_positions=64)
    cache = s.kv_cache(c.Hkv, c.D, 4)
    cache.append(c.past_k[:4 * c.Hkv * c.D].copy(), c.past_v[:4 * c.Hkv * c.D].copy(), 4)
    x = torch.zeros(c.hidden, device="cuda")
    out = torch.zeros(c.hidden, device="cuda")
    layer = AttentionLayer(c.hidden, c.Hq, c.Hkv, c.D, W["q"], W["k"], W["v"], W["o"], rope=table)
    with pytest.raises(sa.ShapeError):  # the cache is full: the append would not fit
        s.attention_sublayer(layer, x, 1, cache, out)
    assert cache.len() == 4
    bad = AttentionLayer(c.hidden, c.Hq, c.Hkv, c.D, W["q"], W["k"], W["v"], W["o"], rope=table, q_prescale=2.0)
    with pytest.raises(sa.ArgumentError):
        s.attention_sublayer(bad, x, 1, None, out)
    swapped = AttentionLayer(c.hidden, c.Hq, c.Hkv, c.D, W["q"], W["k"], W["v"], W["k"], rope=table)
    with pytest.raises(sa.ShapeError):
        s.attention_sublayer(swapped, x, 1, None, out)
    s.sync()


def test_caches_and_weights_outlive_their_session(gpu):
    """Releasing the session first must not invalidate what was created on it
    (the library keeps the session until its last cache and weight are freed)."""
    from spissa_amd import _ffi
    from spissa_amd.device import Session

    s = Session(0)
    cache = s.kv_cache(2, 64, 8)
    w = s.linear_weight(np.zeros(4 * 64, np.float32), 0, 4, 64)
    s.close()  # the caller's reference goes first
    cache.append(np.ones(2 * 64, np.float32), np.ones(2 * 64, np.float32), 1)
    assert cache.len() == 1 and cache.keys().sum() == 128
    lib = _ffi.load()
    lib.spissa_linear_weight_free(w.handle)
    w._h = None
    cache.close()
