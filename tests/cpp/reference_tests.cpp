// reference_tests.cpp -- the reference runtime's own tests for the attention
// path, restated against the C++ API of include/spissa.hpp (which runs them on
// the GPU through libspissa_hip.so). Each test names the Rust test it
// restates (file:line under crates/spissa-runtime/src); the inputs, expected
// values and tolerances are the reference's. Tests marked HOST run no device
// work (argument validation and pure functions); the rest need a GPU.
//
//   reference_tests            run every test
//   reference_tests --host     run only the HOST tests (no GPU needed)
//   reference_tests --list     print the test names
//
// Exit status 0 iff every selected test passed.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "spissa.hpp"

using namespace spissa;

namespace {

struct TestCase {
  const char *name;
  bool host_only;
  std::function<void()> fn;
};

std::vector<TestCase> &registry() {
  static std::vector<TestCase> r;
  return r;
}

struct Register {
  Register(const char *name, bool host_only, std::function<void()> fn) {
    registry().push_back({name, host_only, std::move(fn)});
  }
};

struct Failure {
  std::string what;
};

#define TEST(name) \
  static void name(); \
  static Register reg_##name(#name, false, name); \
  static void name()
#define HOST_TEST(name) \
  static void name(); \
  static Register reg_##name(#name, true, name); \
  static void name()

#define CHECK(cond)                                                                              \
  do {                                                                                           \
    if (!(cond)) throw Failure{std::string(__FILE__ ":") + std::to_string(__LINE__) + ": " #cond}; \
  } while (0)

[[noreturn]] void fail(const std::string &msg) { throw Failure{msg}; }

// rotary.rs:606-614 assert_close_vec
void assert_close_vec(const float *actual, size_t n_actual, const std::vector<float> &expected, float eps) {
  if (n_actual != expected.size())
    fail("length " + std::to_string(n_actual) + " != " + std::to_string(expected.size()));
  for (size_t i = 0; i < n_actual; ++i)
    if (!(std::fabs(actual[i] - expected[i]) <= eps)) {
      char buf[160];
      std::snprintf(buf, sizeof buf, "idx=%zu: actual=%.9g, expected=%.9g (eps %g)", i, actual[i], expected[i], eps);
      fail(buf);
    }
}
void assert_close_vec(const std::vector<float> &actual, const std::vector<float> &expected, float eps) {
  assert_close_vec(actual.data(), actual.size(), expected, eps);
}

template <class T>
T ok(Result<T> r) {
  if (r.is_err()) fail(std::string("unexpected ") + kind_name(r.error().kind) + ": " + r.error().message);
  return std::move(r).unwrap();
}
void ok(Result<void> r) {
  if (r.is_err()) fail(std::string("unexpected ") + kind_name(r.error().kind) + ": " + r.error().message);
}

std::vector<float> slice(const std::vector<float> &v, size_t from, size_t to) {
  return std::vector<float>(v.begin() + from, v.begin() + to);
}

// rotary.rs:616-639 manual_gpt_neox_rotary (f32 throughout, as in Rust).
void manual_gpt_neox_rotary(std::vector<float> &values, const RotaryEmbeddingConfig &config) {
  const size_t half_rotary = config.rotary_dim / 2;
  for (size_t pos = 0; pos < config.seq_len; ++pos) {
    const size_t absolute_pos = config.position_offset + pos;
    for (size_t head = 0; head < config.num_heads; ++head) {
      const size_t row_start = (pos * config.num_heads + head) * config.head_dim;
      for (size_t pair = 0; pair < half_rotary; ++pair) {
        const size_t first_idx = row_start + pair, second_idx = row_start + pair + half_rotary;
        const float first = values[first_idx], second = values[second_idx];
        const float inv_freq = 1.0f / std::pow(config.base, (float)(2 * pair) / (float)config.rotary_dim);
        const float angle = (float)absolute_pos * inv_freq;
        const float c = std::cos(angle), s = std::sin(angle);
        values[first_idx] = first * c - second * s;
        values[second_idx] = second * c + first * s;
      }
    }
  }
}

// ---------------------------------------------------------------- rotary.rs

// rotary.rs:641-670
TEST(gpt_neox_rotary_rotates_first_rotary_dims_and_preserves_tail) {
  const RotaryEmbeddingConfig config{2, 1, 6, 4, 10000.0f, 0};
  std::vector<float> q{1.0, 2.0, 3.0, 4.0, 9.0, 10.0, 0.5, -0.25, 1.5, -2.0, 11.0, 12.0};
  std::vector<float> k{-1.0, 0.75, 2.0, 0.25, 13.0, 14.0, 2.5, -1.5, 0.5, 3.0, 15.0, 16.0};
  auto expected_q = q, expected_k = k;
  manual_gpt_neox_rotary(expected_q, config);
  manual_gpt_neox_rotary(expected_k, config);

  ok(apply_gpt_neox_rotary_inplace(q, k, config));

  assert_close_vec(q, expected_q, 1e-6f);
  assert_close_vec(k, expected_k, 1e-6f);
  CHECK(q[4] == 9.0f);
  CHECK(q[5] == 10.0f);
  CHECK(k[10] == 15.0f);
  CHECK(k[11] == 16.0f);
}

// rotary.rs:672-699 (bitwise: eps 0)
TEST(gemma_local_rotary_with_unit_divisor_matches_llama_rotary) {
  const RotaryEmbeddingConfig config{3, 2, 4, 4, 10000.0f, 1};
  std::vector<float> q(config.seq_len * 2 * config.head_dim), k(config.seq_len * config.head_dim);
  for (size_t i = 0; i < q.size(); ++i) q[i] = ((float)i * 0.1f) - 1.0f;
  for (size_t i = 0; i < k.size(); ++i) k[i] = 0.5f - ((float)i * 0.05f);

  auto q_llama = q, k_llama = k;
  ok(apply_llama_rotary_inplace(q_llama, k_llama, 2, 1, config, nullptr));
  auto q_gemma = q, k_gemma = k;
  ok(apply_gemma_rotary_inplace(q_gemma, k_gemma, 2, 1, config, 1.0f));

  assert_close_vec(q_gemma, q_llama, 0.0f);
  assert_close_vec(k_gemma, k_llama, 0.0f);
}

// rotary.rs:701-754
TEST(gemma_global_rotary_divides_position_by_scaling_factor) {
  const RotaryEmbeddingConfig config{2, 1, 4, 4, 1000000.0f, 3};
  const float factor = 8.0f;
  const std::vector<float> q{1.0, 2.0, 3.0, 4.0, -0.5, 0.25, 0.75, -1.5};
  const std::vector<float> k = q;

  auto expected_q = q, expected_k = k;
  const size_t half = config.rotary_dim / 2;
  for (size_t pos = 0; pos < config.seq_len; ++pos) {
    const float scaled = (float)(config.position_offset + pos) / factor;
    const size_t row = pos * config.head_dim;
    for (size_t pair = 0; pair < half; ++pair) {
      const float inv_freq = 1.0f / std::pow(config.base, (float)(2 * pair) / (float)config.rotary_dim);
      const float angle = scaled * inv_freq;
      const float c = std::cos(angle), s = std::sin(angle);
      for (auto *buf : {&expected_q, &expected_k}) {
        const float a = (*buf)[row + pair], b = (*buf)[row + pair + half];
        (*buf)[row + pair] = a * c - b * s;
        (*buf)[row + pair + half] = b * c + a * s;
      }
    }
  }

  auto q_out = q, k_out = k;
  ok(apply_gemma_rotary_inplace(q_out, k_out, 1, 1, config, factor));
  assert_close_vec(q_out, expected_q, 1e-6f);
  assert_close_vec(k_out, expected_k, 1e-6f);

  auto q_unscaled = q, k_unscaled = k;
  ok(apply_gemma_rotary_inplace(q_unscaled, k_unscaled, 1, 1, config, 1.0f));
  bool differs = false;
  for (size_t i = 0; i < q_out.size(); ++i) differs |= std::fabs(q_out[i] - q_unscaled[i]) > 1e-4f;
  CHECK(differs);  // scaled and unscaled global rotary should differ
}

// rotary.rs:756-769
HOST_TEST(gemma_rotary_rejects_invalid_divisor) {
  const RotaryEmbeddingConfig config{1, 1, 2, 2, 10000.0f, 0};
  std::vector<float> q{1.0, 2.0}, k{1.0, 2.0};
  CHECK(apply_gemma_rotary_inplace(q, k, 1, 1, config, 0.0f).is_err());
  CHECK(q[0] == 1.0f && q[1] == 2.0f && k[0] == 1.0f && k[1] == 2.0f);  // validation precedes mutation
}

// rotary.rs:771-788
TEST(kv_cache_appends_tokens_and_rejects_capacity_overflow_without_mutating) {
  auto cache = ok(KvCache::create(1, 2, 3));
  ok(cache.append(std::vector<float>{1.0, 2.0, 3.0, 4.0}, std::vector<float>{5.0, 6.0, 7.0, 8.0}, 2));

  CHECK(cache.len() == 2);
  CHECK(cache.keys() == (std::vector<float>{1.0, 2.0, 3.0, 4.0}));
  CHECK(cache.values() == (std::vector<float>{5.0, 6.0, 7.0, 8.0}));

  auto err = cache.append(std::vector<float>{9.0, 10.0, 11.0, 12.0}, std::vector<float>{13.0, 14.0, 15.0, 16.0}, 2);
  CHECK(err.is_err());
  CHECK(err.error().kind == ErrorKind::Shape);
  CHECK(cache.len() == 2);
  CHECK(cache.keys() == (std::vector<float>{1.0, 2.0, 3.0, 4.0}));
}

// rotary.rs:790-811
TEST(kv_cache_truncate_rolls_back_len_and_buffers) {
  auto cache = ok(KvCache::create(2, 3, 4));
  ok(cache.append(std::vector<float>{1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0, 8.0, 9.0, 10.0, 11.0, 12.0},
                  std::vector<float>{13.0, 14.0, 15.0, 16.0, 17.0, 18.0, 19.0, 20.0, 21.0, 22.0, 23.0, 24.0}, 2));

  ok(cache.truncate(1));

  CHECK(cache.len() == 1);
  CHECK(cache.keys() == (std::vector<float>{1.0, 2.0, 3.0, 4.0, 5.0, 6.0}));
  CHECK(cache.values() == (std::vector<float>{13.0, 14.0, 15.0, 16.0, 17.0, 18.0}));
  CHECK(cache.resident_bytes() == 48);
}

// rotary.rs:813-824
TEST(kv_cache_truncate_rejects_growth) {
  auto cache = ok(KvCache::create(1, 2, 4));
  ok(cache.append(std::vector<float>{1.0, 2.0}, std::vector<float>{3.0, 4.0}, 1));

  auto result = cache.truncate(2);

  CHECK(result.is_err());
  CHECK(cache.len() == 1);
  CHECK(cache.keys() == (std::vector<float>{1.0, 2.0}));
  CHECK(cache.values() == (std::vector<float>{3.0, 4.0}));
}

// rotary.rs:826-851
TEST(cached_attention_for_next_token_matches_full_causal_attention_last_row) {
  const std::vector<float> q_all{0.2, 0.7, -0.1, 0.4, 0.9, -0.3};
  const std::vector<float> k_all{0.5, -0.2, 0.1, 0.8, -0.4, 0.3};
  const std::vector<float> v_all{1.0, 0.0, -0.5, 2.0, 0.25, -1.0};
  auto full = ok(ops::scaled_dot_product_attention(q_all, k_all, v_all, 3, 1, 2, true));

  auto cache = ok(KvCache::create(1, 2, 3));
  ok(cache.append(slice(k_all, 0, 4), slice(v_all, 0, 4), 2));
  auto qs = slice(q_all, 4, 6), ks = slice(k_all, 4, 6), vs = slice(v_all, 4, 6);
  auto incremental = ok(scaled_dot_product_attention_with_cache(qs, ks, vs, &cache, KvAttentionConfig{1, 1, 1, 2, true}));

  assert_close_vec(incremental, slice(full, 4, 6), 1e-6f);
}

// ------------------------------------------------------------------- ops.rs

// ops.rs:506-513
TEST(rms_norm_scales_by_root_mean_square) {
  const std::vector<float> x{3.0, 4.0}, weight{1.0, 1.0};
  auto out = ok(ops::rms_norm(x, weight, 1, 2, 0.0f));
  const float denom = std::sqrt((9.0f + 16.0f) / 2.0f);
  assert_close_vec(out, {3.0f / denom, 4.0f / denom}, 1e-6f);
}

// ops.rs:515-521 (softmax_rows), through the attention that computes it: with
// head_dim 1 and q = 1 the scores are the keys, and one-hot values read the
// softmax weights back out.
TEST(softmax_rows_is_stable_and_sums_to_one) {
  auto w0 = ok(ops::scaled_dot_product_attention(std::vector<float>{1.0f, 1.0f}, std::vector<float>{1000.0f, 1001.0f},
                                                 std::vector<float>{1.0f, 0.0f}, 2, 1, 1, false));
  auto w1 = ok(ops::scaled_dot_product_attention(std::vector<float>{1.0f, 1.0f}, std::vector<float>{1000.0f, 1001.0f},
                                                 std::vector<float>{0.0f, 1.0f}, 2, 1, 1, false));
  assert_close_vec({w0[0], w1[0]}, {0.26894143f, 0.7310586f}, 1e-6f);
  auto u = ok(ops::scaled_dot_product_attention(std::vector<float>{1.0f, 1.0f}, std::vector<float>{1.0f, 1.0f},
                                                std::vector<float>{1.0f, 0.0f}, 2, 1, 1, false));
  assert_close_vec(u, {0.5f, 0.5f}, 1e-6f);
}

// ops.rs:536-554
TEST(scaled_dot_product_attention_applies_causal_mask) {
  const std::vector<float> q{1.0, 0.0, 0.0, 1.0};
  const std::vector<float> k = q;
  const std::vector<float> v{10.0, 0.0, 0.0, 20.0};
  auto out = ok(ops::scaled_dot_product_attention(q, k, v, 2, 1, 2, true));

  assert_close_vec(out.data(), 2, {10.0f, 0.0f}, 1e-6f);
  CHECK(out[2] > 3.0f && out[2] < 3.4f);
  CHECK(out[3] > 13.0f && out[3] < 13.7f);
}

// ------------------------------------------------------- models, streaming

// models/gemma/model.rs:107-116
HOST_TEST(gemma3_global_layers_are_every_sixth_one_indexed) {
  const size_t pattern = 6;
  std::vector<size_t> globals;
  for (size_t i = 0; i < 34; ++i)
    if (is_global_layer(i, pattern)) globals.push_back(i);
  CHECK(globals == (std::vector<size_t>{5, 11, 17, 23, 29}));
  CHECK(!is_global_layer(33, pattern));
}

// models/gemma/model.rs:118-124
HOST_TEST(degenerate_patterns_make_every_layer_global) {
  for (size_t pattern : {0, 1}) {
    CHECK(is_global_layer(0, pattern));
    CHECK(is_global_layer(7, pattern));
  }
}

// streaming/tests.rs:3731-3813, at the attention level: with identity QKV
// and output projections q = k = v = the input rows, so the streamed layer's
// output is the attention row itself.
TEST(streaming_attention_with_rotary_and_kv_cache_matches_full_decode_last_token) {
  const std::vector<float> previous_input{0.4f, -0.2f, 0.1f, 0.3f};
  const std::vector<float> current_input{0.7f, 0.5f, -0.4f, 0.2f};
  std::vector<float> q = previous_input, k, v;
  q.insert(q.end(), current_input.begin(), current_input.end());
  k = q;
  v = q;
  ok(apply_gpt_neox_rotary_inplace(q, k, RotaryEmbeddingConfig{2, 1, 4, 4, 10000.0f, 0}));
  auto full_attended = ok(ops::scaled_dot_product_attention(q, k, v, 2, 1, 4, true));
  const auto expected = slice(full_attended, 4, 8);

  auto cache = ok(KvCache::create(1, 4, 4));
  ok(cache.append(slice(k, 0, 4), slice(v, 0, 4), 1));
  // The streamed step: project (identity), rotate at position 1, attend over the cache, append.
  std::vector<float> cq = current_input, ck = current_input, cv = current_input;
  ok(apply_gpt_neox_rotary_inplace(cq, ck, RotaryEmbeddingConfig{1, 1, 4, 4, 10000.0f, 1}));
  auto actual = ok(scaled_dot_product_attention_with_cache(cq, ck, cv, &cache, KvAttentionConfig{1, 1, 1, 4, true}));
  ok(cache.append(ck, cv, 1));

  assert_close_vec(actual, expected, 1e-6f);
  CHECK(cache.len() == 2);
  assert_close_vec(cache.keys(), slice(k, 0, 8), 1e-6f);
  assert_close_vec(cache.values(), slice(v, 0, 8), 1e-6f);
}

// tiny.rs:1800-1898 and echo.rs:1247-1355 (prefill then decode steps equal a
// full-context recompute at every step, 1e-5), at the attention level of one
// Llama layer with grouped-query heads.
TEST(prefill_then_decode_steps_match_full_context_recompute) {
  const size_t T = 7, P0 = 3, Hq = 4, Hkv = 2, D = 8;
  std::vector<float> q(T * Hq * D), k(T * Hkv * D), v(T * Hkv * D);
  uint32_t x = 12345u;
  auto draw = [&] {
    x = x * 1664525u + 1013904223u;
    return (float)((x >> 8) & 0xffff) / 32768.0f - 1.0f;
  };
  for (auto *a : {&q, &k, &v})
    for (auto &e : *a) e = draw();
  ok(apply_llama_rotary_inplace(q, k, Hq, Hkv, RotaryEmbeddingConfig{T, Hq, D, D, 500000.0f, 0}, nullptr));

  auto cache = ok(KvCache::create(Hkv, D, T));
  const size_t qw = Hq * D, kw = Hkv * D;
  for (size_t end = P0; end <= T; ++end) {
    const size_t begin = end == P0 ? 0 : end - 1;  // one prefill of P0 tokens, then single-token decode
    auto full = ok(scaled_dot_product_attention_with_cache(slice(q, 0, end * qw), slice(k, 0, end * kw),
                                                           slice(v, 0, end * kw), nullptr,
                                                           KvAttentionConfig{end, Hq, Hkv, D, true}));
    auto qs = slice(q, begin * qw, end * qw), ks = slice(k, begin * kw, end * kw), vs = slice(v, begin * kw, end * kw);
    auto step = ok(scaled_dot_product_attention_with_cache(qs, ks, vs, &cache,
                                                           KvAttentionConfig{end - begin, Hq, Hkv, D, true}));
    ok(cache.append(ks, vs, end - begin));
    assert_close_vec(step, slice(full, begin * qw, end * qw), 1e-5f);
  }
  CHECK(cache.len() == T);
  CHECK(cache.keys() == k);
  CHECK(cache.values() == v);
}

// models/llama/session/tests_core.rs:646-660: a failure after some layers'
// caches were appended rolls every cache back to the pre-call length.
TEST(session_append_rolls_back_all_caches_after_a_later_layer_fails) {
  auto layer0 = ok(KvCache::create(1, 2, 4));
  auto layer1 = ok(KvCache::create(1, 2, 1));
  const std::vector<float> kk{1, 2, 3, 4}, vv{5, 6, 7, 8};
  const size_t before = layer0.len();
  ok(layer0.append(kk, vv, 2));
  auto r = layer1.append(kk, vv, 2);
  CHECK(r.is_err() && r.error().kind == ErrorKind::Shape);
  ok(layer0.truncate(before));
  CHECK(layer0.len() == 0 && layer0.is_empty() && layer0.resident_bytes() == 0);
  CHECK(layer1.len() == 0);
}

// --------------------------------------------------------- streaming linear

// streaming/tests.rs:2128-2181 (raw bf16 batch 1) and 2078-2125 (raw fp16):
// the same 4x3 weight, input [1.5, -2, 0.25], bias; every product and partial
// sum is exact in f32, so the expected values are exact.
static void linear_kat(DType dtype, const std::vector<uint16_t> &bits) {
  LinearModel model;
  model.add("linear.batch1.weight", ok(LinearWeight::create(dtype, 4, 3, bits.data(), bits.size() * 2)));
  const std::vector<float> input{1.5f, -2.0f, 0.25f}, bias{0.0f, 0.5f, -1.0f, 4.0f};
  auto actual = ok(streaming_tile_linear_from_model(model, "linear.batch1.weight", input, &bias,
                                                    StreamingTileLinearConfig{StreamingLinearConfig{1, 3, 4}, 2}));
  assert_close_vec(actual, {3.25f, -2.875f, -1.75f, 5.1875f}, 1e-6f);
}
TEST(streaming_tile_linear_uses_raw_bf16_batch1_path) {
  linear_kat(DType::Bf16, {0x3f00, 0xbf80, 0x4000, 0xc000, 0x3e80, 0x3f00, 0x3f80, 0x3f80, 0xbf80, 0x0000, 0xbf00,
                           0x3f40});
}
TEST(streaming_tile_linear_matches_raw_fp16_batch1_linear) {
  linear_kat(DType::F16, {0x3800, 0xbc00, 0x4000, 0xc000, 0x3400, 0x3800, 0x3c00, 0x3c00, 0xbc00, 0x0000, 0xb800,
                          0x3a00});
}

// ops.rs:488-495 through the device linear with f32 weights
TEST(linear_uses_transposed_weight_layout) {
  const std::vector<float> weight{1.0, 0.0, 1.0, 0.5, 0.5, 0.5}, bias{1.0, -1.0};
  auto w = ok(LinearWeight::create(DType::F32, 2, 3, weight.data(), weight.size() * 4));
  auto out = ok(linear(w, std::vector<float>{1.0f, 2.0f, 3.0f}, &bias, StreamingLinearConfig{1, 3, 2}));
  CHECK(out == (std::vector<float>{5.0f, 2.0f}));
}

// streaming/validation.rs:225-256 and lazy.rs:357-361: errors before any work
HOST_TEST(streaming_tile_linear_rejects_zero_tile_and_missing_tensor) {
  LinearModel model;
  const std::vector<float> input{1.0f, 2.0f, 3.0f};
  auto zero = streaming_tile_linear_from_model(model, "w", input, nullptr,
                                               StreamingTileLinearConfig{StreamingLinearConfig{1, 3, 2}, 0});
  CHECK(zero.is_err() && zero.error().kind == ErrorKind::Shape);
  auto missing = streaming_tile_linear_from_model(model, "w", input, nullptr,
                                                  StreamingTileLinearConfig{StreamingLinearConfig{1, 3, 2}, 4});
  CHECK(missing.is_err() && missing.error().kind == ErrorKind::MissingTensor);
}

TEST(linear_rejects_mismatched_shapes_and_bytes) {
  const std::vector<float> weight(6, 0.0f);
  auto w = ok(LinearWeight::create(DType::F32, 2, 3, weight.data(), weight.size() * 4));
  auto bad_input = linear(w, std::vector<float>(4, 1.0f), nullptr, StreamingLinearConfig{1, 3, 2});
  CHECK(bad_input.is_err() && bad_input.error().kind == ErrorKind::Shape);
  const std::vector<float> bias3(3, 0.0f);
  auto bad_bias = linear(w, std::vector<float>(3, 1.0f), &bias3, StreamingLinearConfig{1, 3, 2});
  CHECK(bad_bias.is_err() && bad_bias.error().kind == ErrorKind::Shape);
  auto bad_shape = linear(w, std::vector<float>(2, 1.0f), nullptr, StreamingLinearConfig{1, 2, 3});
  CHECK(bad_shape.is_err() && bad_shape.error().kind == ErrorKind::Shape);
  auto bad_bytes = LinearWeight::create(DType::F32, 2, 3, weight.data(), 5 * 4);
  CHECK(bad_bytes.is_err() && bad_bytes.error().kind == ErrorKind::InvalidTensorData);
}

// ------------------------------------------- LM head and greedy sampling

// ops.rs:570-573
TEST(sample_argmax_is_deterministic) { CHECK(ok(sample_argmax(std::vector<float>{0.1f, 2.0f, 1.9f})) == 1); }

// ops.rs:575-586
TEST(sample_argmax_excluding_uses_next_best_token) {
  CHECK(ok(sample_argmax_excluding(std::vector<float>{0.1f, 2.0f, 1.9f}, 1)) == 2);
  CHECK(ok(sample_argmax_excluding(std::vector<float>{0.1f, 2.0f, 1.9f}, 99)) == 1);
  CHECK(ok(sample_argmax_excluding(std::vector<float>{2.0f}, 0)) == 0);
}

// ops.rs:309-314: empty logits are InvalidTensorData
TEST(sample_argmax_rejects_empty_logits) {
  auto r = sample_argmax(std::vector<float>{});
  CHECK(r.is_err() && r.error().kind == ErrorKind::InvalidTensorData);
  CHECK(r.error().message.find("cannot sample from empty logits") != std::string::npos);
}

static size_t first_argmax(const std::vector<float> &v) {
  size_t best = 0;
  for (size_t i = 1; i < v.size(); ++i)
    if (v[i] > v[best]) best = i;
  return best;
}

// streaming/tests.rs:303-327: the LM head over an f32 table equals the serial
// left-to-right loop bit for bit (hidden 5 runs the device's sequential kernel)
TEST(r131_parallel_lm_head_matches_serial_bit_for_bit) {
  const size_t hidden = 5, vocab = 37;
  std::vector<float> last_hidden(hidden), weight(vocab * hidden);
  for (size_t h = 0; h < hidden; ++h) last_hidden[h] = std::sin((float)h * 0.37f - 0.5f);
  for (size_t i = 0; i < weight.size(); ++i) weight[i] = std::cos((float)i * 0.013f - 0.21f) * 0.5f;
  auto table = ok(LinearWeight::create(DType::F32, vocab, hidden, weight.data(), weight.size() * 4));
  auto parallel = ok(lm_head_logits_parallel(last_hidden, table, vocab, hidden));
  std::vector<float> serial(vocab);
  for (size_t v = 0; v < vocab; ++v) {
    float sum = 0.0f;
    for (size_t h = 0; h < hidden; ++h) sum += last_hidden[h] * weight[v * hidden + h];
    serial[v] = sum;
  }
  CHECK(std::memcmp(parallel.data(), serial.data(), vocab * 4) == 0);
}

// streaming/tests.rs:329-366: the bf16 table agrees with the f32 table of its
// exact upcast within 1e-4, with the same argmax
TEST(lm_head_bf16_direct_matches_f32_upcast_within_accumulation_tolerance) {
  const size_t hidden = 5, vocab = 37;
  std::vector<float> last_hidden(hidden), f32_weight(vocab * hidden);
  std::vector<uint16_t> bits(vocab * hidden);
  for (size_t h = 0; h < hidden; ++h) last_hidden[h] = std::cos((float)h * 0.41f - 0.6f);
  for (size_t i = 0; i < bits.size(); ++i) {
    const float v = std::sin((float)i * 0.017f - 0.3f) * 0.5f;
    uint32_t u;
    std::memcpy(&u, &v, 4);
    bits[i] = (uint16_t)(u >> 16);
    const uint32_t up = (uint32_t)bits[i] << 16;
    std::memcpy(&f32_weight[i], &up, 4);
  }
  auto tb = ok(LinearWeight::create(DType::Bf16, vocab, hidden, bits.data(), bits.size() * 2));
  auto tf = ok(LinearWeight::create(DType::F32, vocab, hidden, f32_weight.data(), f32_weight.size() * 4));
  auto from_bf16 = ok(lm_head_logits_parallel_bf16(last_hidden, tb, vocab, hidden));
  auto from_f32 = ok(lm_head_logits_parallel(last_hidden, tf, vocab, hidden));
  float max_abs_diff = 0.0f;
  for (size_t v = 0; v < vocab; ++v) max_abs_diff = std::fmax(max_abs_diff, std::fabs(from_bf16[v] - from_f32[v]));
  CHECK(max_abs_diff < 1e-4f);
  CHECK(first_argmax(from_bf16) == first_argmax(from_f32));
  CHECK(ok(sample_argmax(from_bf16)) == first_argmax(from_bf16));
}

// streaming/tests.rs:4093-4153: Gemma 3 4B hidden, vocab 257, xorshift data;
// within 1e-2 of the scalar reference and the same argmax
TEST(lm_head_bf16_simd_matches_scalar_reference_and_preserves_argmax) {
  const size_t hidden = 2560, vocab = 257;
  uint64_t state = 0x9e3779b97f4a7c15ull;
  auto next = [&]() {
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    return (float)(state >> 40) / 16777216.0f - 0.5f;
  };
  std::vector<float> last_hidden(hidden), weight_vals(vocab * hidden);
  for (auto &x : last_hidden) x = next() * 2.0f;
  std::vector<uint16_t> bits(vocab * hidden);
  for (size_t i = 0; i < bits.size(); ++i) {
    const float v = next();
    uint32_t u;
    std::memcpy(&u, &v, 4);
    bits[i] = (uint16_t)(u >> 16);
    const uint32_t up = (uint32_t)bits[i] << 16;
    std::memcpy(&weight_vals[i], &up, 4);
  }
  auto table = ok(LinearWeight::create(DType::Bf16, vocab, hidden, bits.data(), bits.size() * 2));
  auto logits = ok(lm_head_logits_parallel_bf16(last_hidden, table, vocab, hidden));
  std::vector<float> reference(vocab);
  for (size_t row = 0; row < vocab; ++row) {
    float sum = 0.0f;
    for (size_t h = 0; h < hidden; ++h) sum += last_hidden[h] * weight_vals[row * hidden + h];
    reference[row] = sum;
  }
  float max_abs_diff = 0.0f;
  for (size_t v = 0; v < vocab; ++v) max_abs_diff = std::fmax(max_abs_diff, std::fabs(logits[v] - reference[v]));
  CHECK(max_abs_diff < 1e-2f);
  CHECK(first_argmax(logits) == first_argmax(reference));
  CHECK(ok(sample_argmax(logits)) == first_argmax(logits));
}

// The device tail (logits and token in one call) against the drop-in calls.
TEST(device_lm_head_token_matches_dropin_argmax) {
  const size_t hidden = 1152, vocab = 20000;
  std::vector<uint16_t> bits(vocab * hidden);
  std::vector<float> x(hidden);
  uint64_t state = 0x243f6a8885a308d3ull;
  auto next = [&]() {
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    return (float)(state >> 40) / 16777216.0f - 0.5f;
  };
  for (auto &b : bits) {
    const float v = next() * 0.1f;
    uint32_t u;
    std::memcpy(&u, &v, 4);
    b = (uint16_t)(u >> 16);
  }
  for (auto &v : x) v = next();
  auto sess = ok(Session::create());
  auto table = ok(sess.linear_weight(DType::Bf16, vocab, hidden, bits.data(), bits.size() * 2));
  float *d_x = nullptr, *d_logits = nullptr;
  int32_t *d_tok = nullptr;
  CHECK(hipMalloc(&d_x, hidden * 4) == hipSuccess && hipMalloc(&d_logits, vocab * 4) == hipSuccess &&
        hipMalloc(&d_tok, 4) == hipSuccess);
  CHECK(hipMemcpy(d_x, x.data(), hidden * 4, hipMemcpyHostToDevice) == hipSuccess);
  auto host = ok(lm_head_logits_parallel_bf16(x, table, vocab, hidden));
  for (std::optional<size_t> excl : {std::optional<size_t>{}, std::optional<size_t>{first_argmax(host)}}) {
    ok(sess.lm_head(table, d_x, d_logits, d_tok, excl));
    ok(sess.sync());
    std::vector<float> logits(vocab);
    int32_t tok = -1;
    CHECK(hipMemcpy(logits.data(), d_logits, vocab * 4, hipMemcpyDeviceToHost) == hipSuccess);
    CHECK(hipMemcpy(&tok, d_tok, 4, hipMemcpyDeviceToHost) == hipSuccess);
    CHECK(std::memcmp(logits.data(), host.data(), vocab * 4) == 0);
    CHECK((size_t)tok == ok(sample_argmax_excluding(logits, excl)));
  }
  (void)hipFree(d_x);
  (void)hipFree(d_logits);
  (void)hipFree(d_tok);
}

// models/llama/generate.rs:200-450 on the device in one call equals the same
// sequence through the drop-in API: rms_norm, three projections, RoPE at the
// cache's next position, cached attention, append, o projection.
TEST(attention_sublayer_matches_the_dropin_sequence) {
  const size_t H = 256, Hq = 4, Hkv = 2, D = 64, P = 9;
  const float base = 500000.0f, eps = 1e-5f;
  uint32_t st = 7u;
  auto draw = [&](size_t n, float scale) {
    std::vector<float> v(n);
    for (auto &e : v) {
      st = st * 1664525u + 1013904223u;
      e = scale * ((float)((st >> 8) & 0xffff) / 32768.0f - 1.0f);
    }
    return v;
  };
  auto x = draw(H, 1.0f), norm = draw(H, 0.1f), wq = draw(Hq * D * H, 0.05f), wk = draw(Hkv * D * H, 0.05f),
       wv = draw(Hkv * D * H, 0.05f), wo = draw(H * Hq * D, 0.05f), pk = draw(P * Hkv * D, 1.0f),
       pv = draw(P * Hkv * D, 1.0f);
  for (auto &g : norm) g += 1.0f;

  // drop-in sequence on the default session
  auto Wq = ok(LinearWeight::create(DType::F32, Hq * D, H, wq.data(), wq.size() * 4));
  auto Wk = ok(LinearWeight::create(DType::F32, Hkv * D, H, wk.data(), wk.size() * 4));
  auto Wv = ok(LinearWeight::create(DType::F32, Hkv * D, H, wv.data(), wv.size() * 4));
  auto Wo = ok(LinearWeight::create(DType::F32, H, Hq * D, wo.data(), wo.size() * 4));
  auto ref_cache = ok(KvCache::create(Hkv, D, P + 1));
  ok(ref_cache.append(pk, pv, P));
  auto xn = ok(ops::rms_norm(x, norm, 1, H, eps));
  auto q = ok(linear(Wq, xn, nullptr, StreamingLinearConfig{1, H, Hq * D}));
  auto k = ok(linear(Wk, xn, nullptr, StreamingLinearConfig{1, H, Hkv * D}));
  auto v = ok(linear(Wv, xn, nullptr, StreamingLinearConfig{1, H, Hkv * D}));
  ok(apply_llama_rotary_inplace(q, k, Hq, Hkv, RotaryEmbeddingConfig{1, Hq, D, D, base, P}));
  auto att = ok(scaled_dot_product_attention_with_cache(q, k, v, &ref_cache, KvAttentionConfig{1, Hq, Hkv, D, true}));
  ok(ref_cache.append(k, v, 1));
  auto expected = ok(linear(Wo, att, nullptr, StreamingLinearConfig{1, Hq * D, H}));

  // one device call
  auto session = ok(Session::create(0));
  auto sq = ok(session.linear_weight(DType::F32, Hq * D, H, wq.data(), wq.size() * 4));
  auto sk = ok(session.linear_weight(DType::F32, Hkv * D, H, wk.data(), wk.size() * 4));
  auto sv = ok(session.linear_weight(DType::F32, Hkv * D, H, wv.data(), wv.size() * 4));
  auto so = ok(session.linear_weight(DType::F32, H, Hq * D, wo.data(), wo.size() * 4));
  auto cache = ok(session.kv_cache(Hkv, D, P + 1));
  ok(cache.append(pk, pv, P));
  auto table = ok(session.rope_table(RopeKind::Llama, D, base, P + 1));
  float *dx = nullptr, *dnorm = nullptr, *dout = nullptr;
  CHECK(hipMalloc(&dx, H * 4) == hipSuccess && hipMalloc(&dnorm, H * 4) == hipSuccess &&
        hipMalloc(&dout, H * 4) == hipSuccess);
  CHECK(hipMemcpy(dx, x.data(), H * 4, hipMemcpyHostToDevice) == hipSuccess);
  CHECK(hipMemcpy(dnorm, norm.data(), H * 4, hipMemcpyHostToDevice) == hipSuccess);
  AttentionLayer layer{H, Hq, Hkv, D, &sq, &sk, &sv, &so};
  layer.d_input_norm = dnorm;
  layer.eps = eps;
  layer.rope = &table;
  ok(session.attention_sublayer(layer, dx, 1, &cache, dout));
  ok(session.sync());
  std::vector<float> got(H);
  CHECK(hipMemcpy(got.data(), dout, H * 4, hipMemcpyDeviceToHost) == hipSuccess);
  (void)hipFree(dx);
  (void)hipFree(dnorm);
  (void)hipFree(dout);

  float ref_max = 0.0f;
  for (float e : expected) ref_max = std::fmax(ref_max, std::fabs(e));
  assert_close_vec(got, expected, 1e-5f * ref_max);
  CHECK(cache.len() == P + 1);
  const auto ck = cache.keys(), rk = ref_cache.keys();
  float kmax = 0.0f;
  for (float e : rk) kmax = std::fmax(kmax, std::fabs(e));
  assert_close_vec(ck, rk, 1e-5f * kmax);
}

// --------------------------------------------------- ABI contract (no Rust test)

// rotary.rs:17-38: round down to an even count; errors for empty results.
HOST_TEST(gpt_neox_rotary_dim_rounds_down_to_even) {
  CHECK(ok(gpt_neox_rotary_dim(64, 0.25f)) == 16);
  CHECK(ok(gpt_neox_rotary_dim(80, 0.25f)) == 20);
  CHECK(ok(gpt_neox_rotary_dim(6, 0.5f)) == 2);  // 3 -> 2
  CHECK(ok(gpt_neox_rotary_dim(128, 1.0f)) == 128);
  CHECK(gpt_neox_rotary_dim(0, 0.5f).error().kind == ErrorKind::Shape);
  CHECK(gpt_neox_rotary_dim(2, 0.4f).error().kind == ErrorKind::Shape);  // 0.8 -> 0
  CHECK(gpt_neox_rotary_dim(64, 0.0f).is_err());
  CHECK(gpt_neox_rotary_dim(64, 1.5f).is_err());
  CHECK(gpt_neox_rotary_dim(64, NAN).is_err());
}

// rotary.rs:83-96: shape errors before any mutation.
HOST_TEST(llama_rotary_rejects_mismatched_lengths_without_mutating) {
  const RotaryEmbeddingConfig config{2, 2, 4, 4, 10000.0f, 0};
  std::vector<float> q(2 * 2 * 4, 1.0f), k(2 * 1 * 4 + 1, 1.0f);
  auto r = apply_llama_rotary_inplace(q, k, 2, 1, config, nullptr);
  CHECK(r.is_err() && r.error().kind == ErrorKind::Shape);
  for (float e : q) CHECK(e == 1.0f);
}

// #[derive(Clone)] on KvCache (rotary.rs:195): a clone is an independent copy.
TEST(kv_cache_clone_is_independent) {
  auto cache = ok(KvCache::create(1, 2, 4));
  ok(cache.append(std::vector<float>{1, 2}, std::vector<float>{3, 4}, 1));
  auto copy = ok(cache.clone());
  ok(cache.append(std::vector<float>{5, 6}, std::vector<float>{7, 8}, 1));
  CHECK(copy.len() == 1 && cache.len() == 2);
  CHECK(copy.keys() == (std::vector<float>{1, 2}));
  cache.clear();
  CHECK(cache.is_empty() && copy.values() == (std::vector<float>{3, 4}));
}

// Device tier: one fused decode step (RoPE + attention + append in two
// launches) equals the drop-in call sequence of models/llama/generate.rs:383-416
// (RoPE, cached attention, append) at Llama-3.2-1B head geometry.
TEST(fused_decode_step_matches_dropin_sequence) {
  const size_t Hq = 32, Hkv = 8, D = 64, P = 37;
  const float base = 500000.0f;
  auto session = ok(Session::create(0));
  std::vector<float> past_k(P * Hkv * D), past_v(P * Hkv * D), q(Hq * D), k(Hkv * D), v(Hkv * D);
  uint32_t x = 99u;
  for (auto *a : {&past_k, &past_v, &q, &k, &v})
    for (auto &e : *a) {
      x = x * 1664525u + 1013904223u;
      e = (float)((x >> 8) & 0xffff) / 32768.0f - 1.0f;
    }

  // Drop-in sequence on the host API.
  auto ref_cache = ok(KvCache::create(Hkv, D, P + 1));
  ok(ref_cache.append(past_k, past_v, P));
  auto rq = q, rk = k;
  ok(apply_llama_rotary_inplace(rq, rk, Hq, Hkv, RotaryEmbeddingConfig{1, Hq, D, D, base, P}, nullptr));
  auto expected = ok(scaled_dot_product_attention_with_cache(rq, rk, v, &ref_cache, KvAttentionConfig{1, Hq, Hkv, D, true}));
  ok(ref_cache.append(rk, v, 1));

  // Fused step on device buffers.
  auto cache = ok(session.kv_cache(Hkv, D, P + 1));
  ok(cache.append(past_k, past_v, P));
  auto table = ok(session.rope_table(RopeKind::Llama, D, base, P + 1));
  float *dq = nullptr, *dk = nullptr, *dv = nullptr, *dout = nullptr;
  CHECK(hipMalloc(&dq, q.size() * 4) == hipSuccess && hipMalloc(&dk, k.size() * 4) == hipSuccess &&
        hipMalloc(&dv, v.size() * 4) == hipSuccess && hipMalloc(&dout, q.size() * 4) == hipSuccess);
  CHECK(hipMemcpy(dq, q.data(), q.size() * 4, hipMemcpyHostToDevice) == hipSuccess);
  CHECK(hipMemcpy(dk, k.data(), k.size() * 4, hipMemcpyHostToDevice) == hipSuccess);
  CHECK(hipMemcpy(dv, v.data(), v.size() * 4, hipMemcpyHostToDevice) == hipSuccess);
  ok(session.decode_step(&table, dq, dk, dv, {&cache}, KvAttentionConfig{1, Hq, Hkv, D, true}, dout));
  ok(session.sync());
  std::vector<float> got(q.size());
  CHECK(hipMemcpy(got.data(), dout, got.size() * 4, hipMemcpyDeviceToHost) == hipSuccess);
  (void)hipFree(dq);
  (void)hipFree(dk);
  (void)hipFree(dv);
  (void)hipFree(dout);

  float ref_max = 0.0f;
  for (float e : expected) ref_max = std::fmax(ref_max, std::fabs(e));
  assert_close_vec(got, expected, 1e-5f * ref_max);
  CHECK(cache.len() == P + 1);
  CHECK(cache.keys() == ref_cache.keys());  // the appended rotated key is bit-identical
  CHECK(cache.values() == ref_cache.values());
}

}  // namespace

int main(int argc, char **argv) {
  bool host_only = false, list = false;
  for (int i = 1; i < argc; ++i) {
    if (!std::strcmp(argv[i], "--host")) host_only = true;
    else if (!std::strcmp(argv[i], "--list")) list = true;
    else {
      std::fprintf(stderr, "usage: %s [--host] [--list]\n", argv[0]);
      return 2;
    }
  }
  int failed = 0, ran = 0;
  for (auto &t : registry()) {
    if (host_only && !t.host_only) continue;
    if (list) {
      std::printf("%s%s\n", t.name, t.host_only ? " [host]" : "");
      continue;
    }
    ++ran;
    std::printf("test %s ... ", t.name);
    std::fflush(stdout);
    try {
      t.fn();
      std::printf("ok\n");
    } catch (const Failure &f) {
      std::printf("FAILED\n    %s\n", f.what.c_str());
      ++failed;
    } catch (const std::exception &e) {
      std::printf("FAILED\n    exception: %s\n", e.what());
      ++failed;
    }
    std::fflush(stdout);
  }
  if (!list) std::printf("test result: %s. %d passed; %d failed\n", failed ? "FAILED" : "ok", ran - failed, failed);
  return failed ? 1 : 0;
}
