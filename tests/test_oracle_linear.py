"""The CPU oracle's linear projection and weight decoding against the
reference's known-answer tests for them, and against what the mathematics
fixes (exact small-integer products, float64 sums, the IEEE binary16 and
bfloat16 definitions).

Reference tests restated (crates/spissa-runtime/src/...):
  ops.rs:488-495            linear_uses_transposed_weight_layout
  streaming/tests.rs:16-30  bf16_rne_matches_known_values
  streaming/tests.rs:2078-2125, 2128-2181  the raw fp16 / bf16 batch-1 linear
                            KATs (input [1.5, -2, 0.25], 4x3 weight, bias)
"""
import math

import numpy as np
import pytest

import oracle as o
from tests.helpers import assert_bitwise


def f32(x):
    return np.array(x, dtype=np.float32)


def bf16_rne_np(x: np.ndarray) -> np.ndarray:
    """The bf16 round-to-nearest-even bits of a float32 array (no NaNs)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def test_linear_uses_transposed_weight_layout():
    # ops.rs:488-495: input [1,2,3], weight 2x3, bias [1,-1] -> [5, 2] exactly
    out = o.linear(f32([1, 2, 3]), f32([1, 0, 1, 0.5, 0.5, 0.5]), o.DTYPE_F32, f32([1, -1]), 1, 3, 2)
    assert out.tolist() == [5.0, 2.0]


def test_bf16_rne_matches_known_values():
    # streaming/tests.rs:16-30
    assert o.f32_to_bf16_rne(1.0) == 0x3F80
    assert o.f32_to_bf16_rne(0.0) == 0x0000
    tie = np.array([0x3F808000], dtype=np.uint32).view(np.float32)[0]
    above = np.array([0x3F808001], dtype=np.uint32).view(np.float32)[0]
    assert o.f32_to_bf16_rne(float(tie)) == 0x3F80
    assert o.f32_to_bf16_rne(float(above)) == 0x3F81
    n = o.f32_to_bf16_rne(float("nan"))
    assert n & 0x7F80 == 0x7F80 and n & 0x007F != 0


# streaming/tests.rs:2078-2181: the same 4x3 weight as binary16 and bfloat16 bits
FP16_W = [0x3800, 0xBC00, 0x4000, 0xC000, 0x3400, 0x3800, 0x3C00, 0x3C00, 0xBC00, 0x0000, 0xB800, 0x3A00]
BF16_W = [0x3F00, 0xBF80, 0x4000, 0xC000, 0x3E80, 0x3F00, 0x3F80, 0x3F80, 0xBF80, 0x0000, 0xBF00, 0x3F40]
W_VALUES = [0.5, -1.0, 2.0, -2.0, 0.25, 0.5, 1.0, 1.0, -1.0, 0.0, -0.5, 0.75]
KAT_INPUT = [1.5, -2.0, 0.25]
KAT_BIAS = [0.0, 0.5, -1.0, 4.0]
# every product and partial sum is exact in f32: the answer is fixed by arithmetic
KAT_OUT = [3.25, -2.875, -1.75, 5.1875]


@pytest.mark.parametrize("dtype,bits", [(o.DTYPE_F16, FP16_W), (o.DTYPE_BF16, BF16_W)])
def test_raw_16bit_batch1_linear_kat(dtype, bits):
    w = np.array(bits, dtype=np.uint16)
    decode = o.fp16_to_f32 if dtype == o.DTYPE_F16 else o.bf16_to_f32
    assert [decode(b) for b in bits] == W_VALUES
    out = o.linear(f32(KAT_INPUT), w, dtype, f32(KAT_BIAS), 1, 3, 4)
    assert out.tolist() == KAT_OUT
    ref = o.linear(f32(KAT_INPUT), f32(W_VALUES), o.DTYPE_F32, f32(KAT_BIAS), 1, 3, 4)
    assert_bitwise(out, ref, "decoded weights == f32 weights")


def test_fp16_decode_is_ieee_binary16():
    # closed forms of IEEE 754 binary16
    assert o.fp16_to_f32(0x3C00) == 1.0
    assert o.fp16_to_f32(0xC000) == -2.0
    assert o.fp16_to_f32(0x7BFF) == 65504.0
    assert o.fp16_to_f32(0x0400) == 2.0 ** -14          # smallest normal
    assert o.fp16_to_f32(0x0001) == 2.0 ** -24          # smallest subnormal
    assert o.fp16_to_f32(0x03FF) == 1023 * 2.0 ** -24   # largest subnormal
    assert o.fp16_to_f32(0x8000) == 0.0 and math.copysign(1, o.fp16_to_f32(0x8000)) < 0
    assert o.fp16_to_f32(0x7C00) == math.inf and o.fp16_to_f32(0xFC00) == -math.inf
    assert math.isnan(o.fp16_to_f32(0x7E00))
    # every finite code against numpy's float16
    codes = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    ref = codes.view(np.float16).astype(np.float32)
    got = np.array([o.fp16_to_f32(int(c)) for c in codes[::97]], dtype=np.float32)
    fin = np.isfinite(ref[::97])
    assert np.array_equal(got[fin], ref[::97][fin])


def test_bf16_decode_and_rne_round_trip():
    rng = np.random.default_rng(7)
    x = rng.standard_normal(4096).astype(np.float32) * 3
    bits = bf16_rne_np(x)
    for i in range(0, 4096, 131):
        assert o.f32_to_bf16_rne(float(x[i])) == bits[i]
        back = o.bf16_to_f32(int(bits[i]))
        # RNE: the nearest bf16, ties to even; error at most half an ulp of 8 bits
        assert abs(back - x[i]) <= abs(x[i]) * 2.0 ** -8 + 1e-45


@pytest.mark.parametrize("dtype", [o.DTYPE_F32, o.DTYPE_F16, o.DTYPE_BF16])
def test_linear_matches_float64_sums(dtype):
    rng = np.random.default_rng(3)
    B, K, N = 3, 257, 19
    x = rng.standard_normal(B * K).astype(np.float32)
    wf = (rng.standard_normal(N * K) * 0.05).astype(np.float32)
    if dtype == o.DTYPE_F32:
        w, wv = wf, wf.astype(np.float64)
    elif dtype == o.DTYPE_F16:
        h = wf.astype(np.float16)
        w, wv = h.view(np.uint16).copy(), h.astype(np.float64)
    else:
        w = bf16_rne_np(wf)
        wv = (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    bias = rng.standard_normal(N).astype(np.float32)
    out = o.linear(x, w, dtype, bias, B, K, N)
    ref = x.astype(np.float64).reshape(B, K) @ wv.reshape(N, K).T + bias.astype(np.float64)
    # a sequential f32 sum of K terms: error bound ~ K * eps * sum|terms|
    bound = K * 2.0 ** -24 * (np.abs(x.reshape(B, K)) @ np.abs(wv.reshape(N, K)).T + np.abs(bias))
    assert np.all(np.abs(out.reshape(B, N) - ref) <= bound)
    # the oracle's order: bias first, then products in index order, each rounded
    i = 1 * N + 5
    s = np.float32(bias[5])
    for k in range(K):
        s = np.float32(s + np.float32(x[K + k] * np.float32(wv.reshape(N, K)[5, k])))
    assert out[i] == s


def test_linear_rejects_bad_shapes():
    x = f32([1, 2, 3])
    w = f32([1, 0, 1, 0.5, 0.5, 0.5])
    with pytest.raises(o.OracleError) as e:
        o.linear(x, w, o.DTYPE_F32, f32([1, 2, 3]), 1, 3, 2)
    assert e.value.kind == "Shape"
    with pytest.raises(o.OracleError):
        o.linear(f32([1, 2]), w, o.DTYPE_F32, None, 1, 3, 2)
