"""The CPU oracle against every known-answer test the reference holds for this path.

Each test names the reference test it restates (crates/spissa-runtime/src/...).
The reference tests are tiny (head_dim <= 6); the oracle must pass all of
them before any GPU comparison is trusted.
"""
import math

import numpy as np
import pytest

import oracle as o
from tests.helpers import assert_bitwise

pytestmark = pytest.mark.filterwarnings("ignore")


def f32(x):
    return np.array(x, dtype=np.float32)


def manual_rotate_half(values, seq_len, num_heads, head_dim, rotary_dim, base, offset, divisor=None):
    """Restates the reference tests' own hand formula (rotary.rs:616-639, 720-736) in f32."""
    values = values.copy()
    half = rotary_dim // 2
    for pos in range(seq_len):
        absolute = offset + pos
        for head in range(num_heads):
            row = (pos * num_heads + head) * head_dim
            for pair in range(half):
                inv = np.float32(1.0) / np.power(np.float32(base), np.float32(2 * pair) / np.float32(rotary_dim))
                p = np.float32(absolute) if divisor is None else np.float32(absolute) / np.float32(divisor)
                angle = np.float32(p * inv)
                c, s = np.float32(math.cos(angle)), np.float32(math.sin(angle))
                a, b = values[row + pair], values[row + pair + half]
                values[row + pair] = a * c - b * s
                values[row + pair + half] = b * c + a * s
    return values


def test_gpt_neox_rotary_rotates_first_rotary_dims_and_preserves_tail():
    # rotary.rs:642-670
    q = f32([1.0, 2.0, 3.0, 4.0, 9.0, 10.0, 0.5, -0.25, 1.5, -2.0, 11.0, 12.0])
    k = f32([-1.0, 0.75, 2.0, 0.25, 13.0, 14.0, 2.5, -1.5, 0.5, 3.0, 15.0, 16.0])
    eq = manual_rotate_half(q, 2, 1, 6, 4, 10000.0, 0)
    ek = manual_rotate_half(k, 2, 1, 6, 4, 10000.0, 0)
    o.apply_gpt_neox_rotary_inplace(q, k, 2, 1, 6, 4, 10000.0, 0)
    np.testing.assert_allclose(q, eq, atol=1e-6, rtol=0)
    np.testing.assert_allclose(k, ek, atol=1e-6, rtol=0)
    assert q[4] == 9.0 and q[5] == 10.0 and k[10] == 15.0 and k[11] == 16.0


def test_gemma_local_rotary_with_unit_divisor_matches_llama_rotary():
    # rotary.rs:673-699 (exact equality)
    q = (np.arange(3 * 2 * 4, dtype=np.float32) * np.float32(0.1)) - np.float32(1.0)
    k = np.float32(0.5) - (np.arange(3 * 4, dtype=np.float32) * np.float32(0.05))
    ql, kl, qg, kg = q.copy(), k.copy(), q.copy(), k.copy()
    o.apply_llama_rotary_inplace(ql, kl, 2, 1, 3, 4, 4, 10000.0, 1)
    o.apply_gemma_rotary_inplace(qg, kg, 2, 1, 3, 4, 4, 10000.0, 1, 1.0)
    assert_bitwise(qg, ql, "q")
    assert_bitwise(kg, kl, "k")


def test_gemma_global_rotary_divides_position_by_scaling_factor():
    # rotary.rs:702-754
    q = f32([1.0, 2.0, 3.0, 4.0, -0.5, 0.25, 0.75, -1.5])
    k = q.copy()
    eq = manual_rotate_half(q, 2, 1, 4, 4, 1_000_000.0, 3, divisor=8.0)
    qo, ko = q.copy(), k.copy()
    o.apply_gemma_rotary_inplace(qo, ko, 1, 1, 2, 4, 4, 1_000_000.0, 3, 8.0)
    np.testing.assert_allclose(qo, eq, atol=1e-6, rtol=0)
    np.testing.assert_allclose(ko, eq, atol=1e-6, rtol=0)
    qu, ku = q.copy(), k.copy()
    o.apply_gemma_rotary_inplace(qu, ku, 1, 1, 2, 4, 4, 1_000_000.0, 3, 1.0)
    assert np.any(np.abs(qo - qu) > 1e-4)


def test_gemma_rotary_rejects_invalid_divisor():
    # rotary.rs:757-769
    q, k = f32([1.0, 2.0]), f32([1.0, 2.0])
    with pytest.raises(o.OracleError) as e:
        o.apply_gemma_rotary_inplace(q, k, 1, 1, 1, 2, 2, 10000.0, 0, 0.0)
    assert e.value.kind == "InvalidTensorData"


def test_kv_cache_appends_tokens_and_rejects_capacity_overflow_without_mutating():
    # rotary.rs:772-788
    c = o.KvCache(1, 2, 3)
    c.append(f32([1, 2, 3, 4]), f32([5, 6, 7, 8]), 2)
    assert c.len() == 2
    assert list(c.keys()) == [1, 2, 3, 4] and list(c.values()) == [5, 6, 7, 8]
    with pytest.raises(o.OracleError) as e:
        c.append(f32([9, 10, 11, 12]), f32([13, 14, 15, 16]), 2)
    assert e.value.kind == "Shape"
    assert c.len() == 2 and list(c.keys()) == [1, 2, 3, 4]


def test_kv_cache_truncate_rolls_back_len_and_buffers():
    # rotary.rs:791-811
    c = o.KvCache(2, 3, 4)
    c.append(np.arange(1, 13, dtype=np.float32), np.arange(13, 25, dtype=np.float32), 2)
    c.truncate(1)
    assert c.len() == 1
    assert list(c.keys()) == [1, 2, 3, 4, 5, 6]
    assert list(c.values()) == [13, 14, 15, 16, 17, 18]
    assert c.resident_bytes() == 48


def test_kv_cache_truncate_rejects_growth():
    # rotary.rs:814-824
    c = o.KvCache(1, 2, 4)
    c.append(f32([1, 2]), f32([3, 4]), 1)
    with pytest.raises(o.OracleError):
        c.truncate(2)
    assert c.len() == 1 and list(c.keys()) == [1, 2] and list(c.values()) == [3, 4]


def test_cached_attention_for_next_token_matches_full_causal_attention_last_row():
    # rotary.rs:827-851 (the reference allows 1e-6; the restatement is bitwise here)
    q_all = f32([0.2, 0.7, -0.1, 0.4, 0.9, -0.3])
    k_all = f32([0.5, -0.2, 0.1, 0.8, -0.4, 0.3])
    v_all = f32([1.0, 0.0, -0.5, 2.0, 0.25, -1.0])
    full = o.scaled_dot_product_attention(q_all, k_all, v_all, 3, 1, 2, True)
    c = o.KvCache(1, 2, 3)
    c.append(k_all[:4].copy(), v_all[:4].copy(), 2)
    inc = o.sdpa_with_cache(q_all[4:].copy(), k_all[4:].copy(), v_all[4:].copy(), c, 1, 1, 1, 2, True)
    np.testing.assert_allclose(inc, full[4:], atol=1e-6, rtol=0)
    assert_bitwise(inc, full[4:], "decode vs full recompute")


def test_rms_norm_scales_by_root_mean_square():
    # ops.rs:507-513
    out = o.rms_norm(f32([3.0, 4.0]), f32([1.0, 1.0]), 1, 2, 0.0)
    denom = np.sqrt(np.float32(12.5), dtype=np.float32)
    np.testing.assert_allclose(out, [3.0 / denom, 4.0 / denom], atol=1e-6, rtol=0)


def test_softmax_rows_is_stable_and_sums_to_one():
    # ops.rs:516-521
    out = o.softmax_rows(f32([1000.0, 1001.0, 1.0, 1.0]), 2, 2)
    np.testing.assert_allclose(out[:2], [0.26894143, 0.7310586], atol=1e-6, rtol=0)
    np.testing.assert_allclose(out[2:], [0.5, 0.5], atol=1e-6, rtol=0)


def test_scaled_dot_product_attention_applies_causal_mask():
    # ops.rs:537-554, plus the closed form of row 1:
    # scores [1, 0]/sqrt(2) -> p0 = 1/(1+e^{-1/sqrt 2}); out = [10 p0, 20 (1-p0)].
    q = f32([1.0, 0.0, 0.0, 1.0])
    v = f32([10.0, 0.0, 0.0, 20.0])
    out = o.scaled_dot_product_attention(q, q.copy(), v, 2, 1, 2, True)
    np.testing.assert_allclose(out[:2], [10.0, 0.0], atol=1e-6, rtol=0)
    assert 3.0 < out[2] < 3.4 and 13.0 < out[3] < 13.7
    p0 = 1.0 / (1.0 + math.exp(-1.0 / math.sqrt(2.0)))
    np.testing.assert_allclose(out[2:], [10.0 * (1 - p0), 20.0 * p0], rtol=2e-7)


def test_gemma3_global_layers_are_every_sixth_one_indexed():
    # models/gemma/model.rs:107-116 and 118-124
    assert [i for i in range(34) if o.is_global_layer(i, 6)] == [5, 11, 17, 23, 29]
    assert not o.is_global_layer(33, 6)
    for pattern in (0, 1):
        assert o.is_global_layer(0, pattern) and o.is_global_layer(7, pattern)


def test_streaming_attention_with_rotary_and_kv_cache_matches_full_decode_last_token():
    # streaming/tests.rs:3732-3813: NeoX RoPE over 2 tokens, then the cached
    # decode of token 1 equals row 1 of the full causal attention, and the
    # cache holds exactly the rotated K/V rows.
    prev, cur = f32([0.4, -0.2, 0.1, 0.3]), f32([0.7, 0.5, -0.4, 0.2])
    x = np.concatenate([prev, cur])  # identity QKV projection: q = k = v = x
    q, k, v = x.copy(), x.copy(), x.copy()
    o.apply_gpt_neox_rotary_inplace(q, k, 2, 1, 4, 4, 10000.0, 0)
    full = o.scaled_dot_product_attention(q, k, v, 2, 1, 4, True)
    c = o.KvCache(1, 4, 4)
    c.append(k[:4].copy(), v[:4].copy(), 1)
    q1, k1 = cur.copy(), cur.copy()
    o.apply_gpt_neox_rotary_inplace(q1, k1, 1, 1, 4, 4, 10000.0, 1)
    got = o.sdpa_with_cache(q1, k1, cur.copy(), c, 1, 1, 1, 4, True)
    c.append(k1, cur.copy(), 1)
    np.testing.assert_allclose(got, full[4:8], atol=1e-6, rtol=0)
    assert c.len() == 2
    np.testing.assert_allclose(c.keys(), k, atol=1e-6, rtol=0)
    np.testing.assert_allclose(c.values(), v, atol=1e-6, rtol=0)


def test_gpt_neox_rotary_dim_matches_reference_contract():
    # rotary.rs:17-38
    assert o.gpt_neox_rotary_dim(64, 0.25) == 16
    assert o.gpt_neox_rotary_dim(6, 0.5) == 2  # 3 -> odd -> 2
    with pytest.raises(o.OracleError) as e:
        o.gpt_neox_rotary_dim(64, 0.0)
    assert e.value.kind == "InvalidTensorData"
    with pytest.raises(o.OracleError) as e:
        o.gpt_neox_rotary_dim(0, 0.5)
    assert e.value.kind == "Shape"
    with pytest.raises(o.OracleError) as e:
        o.gpt_neox_rotary_dim(1, 0.5)
    assert e.value.kind == "Shape"
