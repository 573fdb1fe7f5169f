"""The CPU oracle's LM head and greedy sampling against the reference's
known-answer tests and against what the mathematics fixes (numpy's argmax,
which returns the first maximal index, float64 dot products, the exact
bf16 -> f32 upcast, and answers derived by hand from IEEE comparisons for the
NaN and signed-zero cases).

Reference tests restated (crates/spissa-runtime/src/...):
  ops.rs:570-573               sample_argmax_is_deterministic
  ops.rs:575-586               sample_argmax_excluding_uses_next_best_token
  streaming/tests.rs:303-327   r131_parallel_lm_head_matches_serial_bit_for_bit
  streaming/tests.rs:329-366   lm_head_bf16_direct_matches_f32_upcast_within_accumulation_tolerance
  streaming/tests.rs:4093-4153 lm_head_bf16_simd_matches_scalar_reference_and_preserves_argmax
"""
import numpy as np
import pytest

import oracle as o

NAN = float("nan")


def f32(x):
    return np.array(x, dtype=np.float32)


def test_sample_argmax_is_deterministic():
    assert o.sample_argmax([0.1, 2.0, 1.9]) == 1


def test_sample_argmax_excluding_uses_next_best_token():
    assert o.sample_argmax_excluding([0.1, 2.0, 1.9], 1) == 2
    assert o.sample_argmax_excluding([0.1, 2.0, 1.9], 99) == 1
    assert o.sample_argmax_excluding([2.0], 0) == 0
    assert o.sample_argmax_excluding([0.1, 2.0, 1.9], None) == 1


def test_empty_logits_are_invalid_tensor_data():
    for call in (lambda: o.sample_argmax([]), lambda: o.sample_argmax_excluding([], 0),
                 lambda: o.sample_argmax_excluding([], None)):
        with pytest.raises(o.OracleError) as e:
            call()
        assert e.value.kind == "InvalidTensorData" and "empty logits" in str(e.value)


@pytest.mark.parametrize("seed", range(6))
def test_argmax_is_numpy_first_argmax(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 5000))
    # few distinct values: many ties, so the first index must win
    x = rng.integers(-3, 4, size=n).astype(np.float32)
    assert o.sample_argmax(x) == int(np.argmax(x))
    e = int(rng.integers(0, n))
    if n > 1:
        rest = np.delete(x, e)
        j = int(np.argmax(rest))
        assert o.sample_argmax_excluding(x, e) == (j if j < e else j + 1)
    else:
        assert o.sample_argmax_excluding(x, e) == 0


def test_argmax_signed_zero_and_infinities():
    # -0.0 == +0.0 under IEEE comparison: the earlier one stays
    assert o.sample_argmax([-0.0, 0.0]) == 0
    assert o.sample_argmax([0.0, -0.0]) == 0
    assert o.sample_argmax([-np.inf, -np.inf]) == 0
    assert o.sample_argmax([-np.inf, -1e38, np.inf, np.inf]) == 2
    assert o.sample_argmax_excluding([np.inf, -np.inf, -np.inf], 0) == 1


def test_argmax_nan_known_answers():
    # `value > best` is false for every comparison with a NaN: a NaN at index 0
    # stays, NaNs elsewhere are never taken
    assert o.sample_argmax([NAN, 5.0, 6.0]) == 0
    assert o.sample_argmax([1.0, NAN, 3.0, NAN]) == 2
    assert o.sample_argmax([1.0, NAN, NAN]) == 0
    # `value <= best` is false whenever a NaN is involved: a NaN replaces the
    # best, and the element after a NaN replaces it
    assert o.sample_argmax_excluding([1.0, NAN, 0.5, 0.2], 3) == 2
    assert o.sample_argmax_excluding([3.0, NAN, 1.0, 2.0], 0) == 3
    assert o.sample_argmax_excluding([5.0, 1.0, NAN], 1) == 2
    assert o.sample_argmax_excluding([NAN, 1.0, 9.0, 4.0], 3) == 2
    assert o.sample_argmax_excluding([9.0, NAN, 1.0, 0.5], 0) == 2
    # an excluded NaN is skipped entirely
    assert o.sample_argmax_excluding([1.0, NAN, 3.0], 1) == 2


def _r131_inputs():
    hidden, vocab = 5, 37
    h = np.arange(hidden, dtype=np.float32)
    last = np.sin(h * np.float32(0.37) - np.float32(0.5)).astype(np.float32)
    i = np.arange(vocab * hidden, dtype=np.float32)
    w = (np.cos(i * np.float32(0.013) - np.float32(0.21)) * np.float32(0.5)).astype(np.float32)
    return last, w, vocab, hidden


def test_lm_head_matches_float64_dot_within_rounding():
    last, w, vocab, hidden = _r131_inputs()
    got = o.lm_head_logits(last, w, o.DTYPE_F32, vocab, hidden)
    want = w.reshape(vocab, hidden).astype(np.float64) @ last.astype(np.float64)
    bound = np.abs(w.reshape(vocab, hidden).astype(np.float64)) @ np.abs(last.astype(np.float64))
    assert np.all(np.abs(got - want) <= 2 * hidden * 2.0 ** -24 * bound)


def test_lm_head_sums_left_to_right_from_zero():
    # 1e8 + 1 rounds back to 1e8 in f32, so only the left-to-right order gives 0
    last = f32([1e8, 1.0, -1e8])
    table = f32([1, 1, 1, 1, -1, 1])
    assert o.lm_head_logits(last, table, o.DTYPE_F32, 2, 3).tolist() == [0.0, 0.0]
    # a product equal to -0.0 added to the starting +0.0 gives +0.0
    z = o.lm_head_logits(f32([-0.0]), f32([1.0]), o.DTYPE_F32, 1, 1)
    assert z[0] == 0.0 and not np.signbit(z[0])


def test_lm_head_bf16_equals_f32_upcast():
    # streaming/tests.rs:329-366: the bf16 table upcasts exactly, so the serial
    # bf16 and f32 paths agree bit for bit
    hidden, vocab = 5, 37
    last = np.cos(np.arange(hidden, dtype=np.float32) * np.float32(0.41) - np.float32(0.6)).astype(np.float32)
    src = (np.sin(np.arange(vocab * hidden, dtype=np.float32) * np.float32(0.017) - np.float32(0.3))
           * np.float32(0.5)).astype(np.float32)
    bits = (src.view(np.uint32) >> 16).astype(np.uint16)
    up = (bits.astype(np.uint32) << 16).view(np.float32)
    a = o.lm_head_logits(last, bits, o.DTYPE_BF16, vocab, hidden)
    b = o.lm_head_logits(last, up, o.DTYPE_F32, vocab, hidden)
    assert a.tobytes() == b.tobytes()


def _xorshift_stream(n, state=0x9E3779B97F4A7C15):
    """streaming/tests.rs:4100-4106: xorshift64 -> ((state >> 40) / 2^24) - 0.5"""
    m = (1 << 64) - 1
    out = np.empty(n, dtype=np.float32)
    for i in range(n):
        state ^= (state << 13) & m
        state ^= state >> 7
        state ^= (state << 17) & m
        out[i] = np.float32(np.float32(state >> 40) / np.float32(16777216.0)) - np.float32(0.5)
    return out


def test_lm_head_bf16_matches_scalar_reference_and_preserves_argmax():
    # streaming/tests.rs:4093-4153 at its own shape (hidden 2560, vocab 257)
    hidden, vocab = 2560, 257
    vals = _xorshift_stream(hidden + vocab * hidden)
    last = (vals[:hidden] * np.float32(2.0)).astype(np.float32)
    bits = (vals[hidden:].view(np.uint32) >> 16).astype(np.uint16)
    got = o.lm_head_logits(last, bits, o.DTYPE_BF16, vocab, hidden)
    wf = (bits.astype(np.uint32) << 16).view(np.float32).reshape(vocab, hidden).astype(np.float64)
    want = wf @ last.astype(np.float64)
    assert np.max(np.abs(got - want)) < 1e-2
    assert o.sample_argmax(got) == int(np.argmax(want))


def test_lm_head_rejects_other_dtypes_and_shapes():
    with pytest.raises(o.OracleError) as e:
        o.lm_head_logits(f32([1.0]), np.zeros(1, np.uint16), o.DTYPE_F16, 1, 1)
    assert e.value.kind == "InvalidTensorData"
