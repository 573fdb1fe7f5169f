"""GPU parity of the LM head (streaming/mod.rs:186-287) and of greedy sampling
(ops.rs:309-348) through the C ABI, against the CPU oracle.

- Logits: the tied-embedding tables of the BASELINE models (vocabulary 262144
  for Gemma 3, 128256 for Llama 3.2) in bf16, plus f32 tables and the
  reference tests' own shapes. Each logit must lie within
  1e-5 * sum_h |x_h w_vh| of the oracle's serial sum (the two differ only in
  f32 summation order).
- Argmax: bit-exact. The device token must equal the oracle's
  sample_argmax / sample_argmax_excluding over the same logits, for ties,
  signed zeros, infinities, NaNs (every position rule of the reference's
  scans), exclusions, unaligned buffers and sizes that span one or many
  partial ranges. For the whole LM head, the token's oracle logit must be
  within the logit tolerance of the oracle's maximum.
"""
import ctypes as C
import zlib

import numpy as np
import pytest

import oracle as o
import spissa_amd as sa
from spissa_amd import _ffi
from spissa_amd.errors import InvalidTensorDataError, ShapeError
from spissa_amd.linear import DTYPE_BF16, DTYPE_F16, DTYPE_F32

pytestmark = pytest.mark.gpu

NAN = float("nan")
LOGIT_TOL = 1e-5  # of sum_h |x_h w_vh|

# (vocab, hidden) of the tied LM heads of the BASELINE models
TABLES = {
    "gemma3_1b": (262144, 1152),
    "gemma3_4b": (262144, 2560),
    "llama32_1b": (128256, 2048),
    "llama32_3b": (128256, 3072),
}


def rng_for(*key) -> np.random.Generator:
    return np.random.default_rng(zlib.crc32(repr(key).encode()))


def table_data(vocab, hidden, dtype, tag):
    """N(0, 0.02) weights drawn on the device (host generation of a 262144 x 2560
    table takes a minute). Returns the table's element data as a host array and
    as a device tensor, and its f32 values on the device."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(zlib.crc32(repr(("table", vocab, hidden, tag)).encode()))
    w = torch.randn(vocab * hidden, generator=g, device="cuda") * 0.02
    if dtype == DTYPE_F32:
        return w.cpu().numpy(), w, w
    b = w.to(torch.bfloat16)
    return b.view(torch.int16).cpu().numpy().view(np.uint16), b, b.to(torch.float32)


def abs_bound(wf, x, vocab, hidden):
    """sum_h |x_h w_vh| per logit (on the device)."""
    import torch

    xa = torch.from_numpy(np.abs(x)).to(wf.device)
    return (wf.view(vocab, hidden).abs() @ xa).double().cpu().numpy()


def check_logits(got, ref, bound, what):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    worst = float(np.max(err / np.maximum(bound, 1e-30)))
    print(f"[lm_head] {what}: max err / bound {worst:.2e}", flush=True)
    assert np.all(err <= LOGIT_TOL * bound + 1e-30), f"{what}: {worst}"


def check_token(tok, ref_logits, bound, what):
    best = int(np.argmax(ref_logits))
    gap_ok = ref_logits[tok] >= ref_logits[best] - 2 * LOGIT_TOL * max(bound[tok], bound[best])
    assert gap_ok, f"{what}: token {tok} logit {ref_logits[tok]} vs max {ref_logits[best]} at {best}"


def dev(a, dtype=None):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda") if dtype is None else \
        torch.tensor(a, dtype=dtype, device="cuda")


def device_argmax(sess, x: np.ndarray, excluded=None, offset=0) -> int:
    """Runs the device argmax over x placed `offset` floats into a buffer."""
    import torch

    buf = torch.zeros(x.size + offset + 1, dtype=torch.float32, device="cuda")
    buf[offset:offset + x.size] = torch.from_numpy(x).to("cuda")
    view = buf[offset:offset + x.size] if x.size else buf[offset:offset + 1]
    tok = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    sess.argmax(view, x.size, tok, excluded)
    sess.sync()
    return int(tok.item())


@pytest.fixture(scope="module")
def sess(gpu):
    """A session on a torch stream that is current for the module's tests, so
    torch's copies and fills are ordered with the session's kernels."""
    import torch

    from spissa_amd.device import Session

    st = torch.cuda.Stream()
    s = Session(0, stream=st)
    with torch.cuda.stream(st):
        yield s
    s.close()


def crafted_cases():
    rng = rng_for("crafted")
    cases = {
        "kat": np.array([0.1, 2.0, 1.9], np.float32),
        "single": np.array([-3.0], np.float32),
        "nan_first": np.array([NAN, 5.0, 6.0], np.float32),
        "nan_middle": np.array([1.0, NAN, 3.0, NAN], np.float32),
        "nan_after_max": np.array([1.0, NAN, 0.5, 0.2], np.float32),
        "all_nan": np.full(9, NAN, np.float32),
        "zeros_signed": np.array([-0.0, 0.0, -0.0], np.float32),
        "zeros_signed2": np.array([0.0, -0.0], np.float32),
        "all_neg_inf": np.full(2050, -np.inf, np.float32),
        "pos_inf_ties": np.array([1.0, np.inf, 2.0, np.inf], np.float32),
    }
    for n in (2, 3, 5, 1023, 1024, 1025, 4097, 128256, 262144, (1 << 20) + 5, 3_000_001):
        cases[f"ties_{n}"] = rng.integers(-4, 5, size=n).astype(np.float32)
        cases[f"normal_{n}"] = rng.standard_normal(n, dtype=np.float32)
    last = rng.standard_normal(262144, dtype=np.float32)
    last[-1] = 100.0
    cases["max_last"] = last
    nan_late = rng.standard_normal((1 << 20) + 5, dtype=np.float32)
    nan_late[rng.integers(0, nan_late.size, 40)] = NAN
    nan_late[700_000] = NAN  # a NaN in a late range, then the suffix spans ranges
    nan_late[900_000] = 50.0
    cases["nan_sprinkled"] = nan_late
    tail_nan = rng.standard_normal(5000, dtype=np.float32)
    tail_nan[-1] = NAN
    cases["nan_last"] = tail_nan
    return cases


CASES = crafted_cases()


def exclusions(x):
    n = x.size
    # none, both ends, past the end, the middle, the maximum itself
    return [None, 0, n - 1, n, n + 5, n // 2, int(np.argmax(np.where(np.isnan(x), -np.inf, x)))]


@pytest.mark.parametrize("name", sorted(CASES))
def test_device_argmax_matches_oracle(sess, name):
    x = CASES[name]
    for excl in exclusions(x):
        want = o.sample_argmax(x) if excl is None else o.sample_argmax_excluding(x, excl)
        for offset in (0, 1):
            got = device_argmax(sess, x, excl, offset)
            assert got == want, f"{name} n={x.size} excluded={excl} offset={offset}: {got} != {want}"


def test_host_sample_argmax_matches_oracle(gpu):
    for name in ("kat", "nan_first", "nan_after_max", "ties_4097", "normal_262144", "zeros_signed"):
        x = CASES[name]
        assert sa.sample_argmax(x) == o.sample_argmax(x), name
        for e in exclusions(x):
            if e is not None:
                assert sa.sample_argmax_excluding(x, e) == o.sample_argmax_excluding(x, e), (name, e)
    # ops.rs:570-586
    assert sa.sample_argmax([0.1, 2.0, 1.9]) == 1
    assert sa.sample_argmax_excluding([0.1, 2.0, 1.9], 1) == 2
    assert sa.sample_argmax_excluding([0.1, 2.0, 1.9], 99) == 1
    assert sa.sample_argmax_excluding([2.0], 0) == 0


def test_empty_logits_are_invalid(gpu, sess):
    import torch

    for call in (lambda: sa.sample_argmax([]), lambda: sa.sample_argmax_excluding([], 0)):
        with pytest.raises(InvalidTensorDataError, match="empty logits"):
            call()
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(InvalidTensorDataError, match="empty logits"):
        sess.argmax(torch.zeros(1, device="cuda"), 0, tok)


@pytest.mark.parametrize("vocab,hidden,dtype,tag", [
    (37, 5, DTYPE_F32, "r131"),            # streaming/tests.rs:303-327 shape (generic kernel)
    (37, 5, DTYPE_BF16, "r131_bf16"),      # streaming/tests.rs:329-366 shape
    (257, 2560, DTYPE_BF16, "simd_4094"),  # streaming/tests.rs:4093-4153 shape
    (1000, 7, DTYPE_BF16, "odd_hidden"),
    (32000, 2048, DTYPE_F32, "f32_table"),
    *[(v, h, DTYPE_BF16, k) for k, (v, h) in TABLES.items()],
])
def test_lm_head_logits_and_token(gpu, sess, vocab, hidden, dtype, tag):
    import torch

    data, d_data, wf = table_data(vocab, hidden, dtype, tag)
    x = rng_for("hidden", vocab, hidden, tag).standard_normal(hidden, dtype=np.float32)
    ref = o.lm_head_logits(x, data, dtype, vocab, hidden)
    bound = abs_bound(wf, x, vocab, hidden)
    del wf
    # large tables upload from device memory, small ones from the host
    table = sess.linear_weight(d_data if vocab * hidden > 1 << 24 else data, dtype, vocab, hidden)
    del d_data
    try:
        # drop-in (host buffers)
        fn = sa.lm_head_logits_parallel if dtype == DTYPE_F32 else sa.lm_head_logits_parallel_bf16
        host = fn(x, table, vocab, hidden)
        check_logits(host, ref, bound, f"{tag} drop-in")
        # device form with the token
        d_logits = torch.empty(vocab, dtype=torch.float32, device="cuda")
        tok = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        for excl in (None, int(np.argmax(ref))):
            sess.lm_head(table, dev(x), d_logits, tok, excl)
            sess.sync()
            got = d_logits.cpu().numpy()
            check_logits(got, ref, bound, f"{tag} device")
            t = int(tok.item())
            want = o.sample_argmax(got) if excl is None else o.sample_argmax_excluding(got, excl)
            assert t == want, f"{tag} excluded={excl}: token {t} != oracle argmax of the same logits {want}"
            if excl is None:
                check_token(t, ref, bound, tag)
        # logits only
        d2 = torch.zeros(vocab, dtype=torch.float32, device="cuda")
        sess.lm_head(table, dev(x), d2)
        sess.sync()
        assert torch.equal(d2, d_logits)
    finally:
        table.close()


def test_lm_head_repeated_rows_tie_to_first(gpu, sess):
    # identical table rows give bitwise identical logits: the first must win
    import torch

    vocab, hidden = 4096, 1152
    rng = rng_for("tie_rows")
    rows = (rng.standard_normal(64 * hidden, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)
    data = np.tile(rows, vocab // 64)
    x = rng.standard_normal(hidden, dtype=np.float32)
    table = sess.linear_weight(data, DTYPE_BF16, vocab, hidden)
    try:
        logits = torch.empty(vocab, dtype=torch.float32, device="cuda")
        tok = torch.zeros(1, dtype=torch.int32, device="cuda")
        sess.lm_head(table, dev(x), logits, tok)
        sess.sync()
        got = logits.cpu().numpy()
        assert int(tok.item()) == o.sample_argmax(got) < 64
        assert np.array_equal(got[:64].view(np.uint32), got[64:128].view(np.uint32))
    finally:
        table.close()


def test_lm_head_errors(gpu, sess):
    data = table_data(16, 8, DTYPE_BF16, "err")[0]
    table = sess.linear_weight(data, DTYPE_BF16, 16, 8)
    f16 = sess.linear_weight(np.zeros(16 * 8, np.uint16), DTYPE_F16, 16, 8)
    lib = _ffi.load()
    try:
        x = np.ones(8, np.float32)
        out = np.empty(16, np.float32)
        fp = lambda a: a.ctypes.data_as(_ffi.c_float_p)  # noqa: E731
        with pytest.raises(ShapeError):
            sa.errors.check(lib.spissa_lm_head_logits(table.handle, fp(x), 7, fp(out), 16))
        with pytest.raises(ShapeError):
            sa.errors.check(lib.spissa_lm_head_logits(table.handle, fp(x), 8, fp(out), 15))
        with pytest.raises(InvalidTensorDataError):
            sa.errors.check(lib.spissa_lm_head_logits(f16.handle, fp(x), 8, fp(out), 16))
        with pytest.raises(ShapeError):
            sa.lm_head_logits_parallel_bf16(x, table, 16, 9)
        with pytest.raises(TypeError):
            sa.lm_head_logits_parallel(x, table, 16, 8)
        assert lib.spissa_lm_head_logits(table.handle, fp(x), 8, fp(out), 16) == 0
    finally:
        f16.close()
        table.close()
