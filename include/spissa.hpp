// spissa.hpp -- C++17 mirror of the Spissa runtime's attention API
// (crates/spissa-runtime/src/rotary.rs, ops.rs, models/gemma/model.rs) and of
// the streaming linear projections either side of it (streaming/linear.rs),
// the LM head and greedy sampling (streaming/mod.rs, ops.rs) over the C ABI
// of spissa_hip.h. Header-only; link with libspissa_hip.so.
//
// The names, argument order and meaning follow the Rust functions they
// replace, so code (and tests) written against the reference read the same:
//   Rust                                        C++
//   Result<T> / RuntimeError::{Shape, ..}      spissa::Result<T> / spissa::RuntimeError
//   &[f32] / &mut [f32]                        spissa::Slice<const float> / Slice<float>
//                                              (from std::vector, or pointer + length)
//   KvCache::new(h, d, max)                    spissa::KvCache::create(h, d, max)
//   Option<&KvCache>                           const spissa::KvCache* (nullptr = None)
//   Option<&[f32]>                             const std::vector<float>* (nullptr = None)
//   Option<usize>                              std::optional<size_t>
//   LazySpissaModel + weight name              spissa::LinearModel (resident weights by name)
// Errors are returned, never thrown; Result<T>::unwrap() throws
// std::runtime_error for callers that prefer exceptions (as .unwrap() panics).
// The drop-in calls copy host buffers to the device and back and return when
// the results are on the host, like the reference's synchronous calls; the
// device tier (Session, RopeTable, decode_step) works on device pointers.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <optional>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "spissa_hip.h"

namespace spissa {

// crates/spissa-runtime/src/error.rs:6-54, the variants this path returns
// (Device and Argument have no reference counterpart: HIP failures and null
// handles; MissingTensor is lazy.rs:357-361).
enum class ErrorKind { Shape, InvalidTensorData, Device, Argument, MissingTensor };

struct RuntimeError {
  ErrorKind kind;
  std::string message;
};

inline const char *kind_name(ErrorKind k) {
  switch (k) {
    case ErrorKind::Shape: return "Shape";
    case ErrorKind::InvalidTensorData: return "InvalidTensorData";
    case ErrorKind::Device: return "Device";
    case ErrorKind::MissingTensor: return "MissingTensor";
    default: return "Argument";
  }
}

template <class T>
class [[nodiscard]] Result {
 public:
  Result(T value) : ok_(true), value_(std::move(value)) {}
  Result(RuntimeError err) : ok_(false), err_(std::move(err)) {}
  bool is_ok() const { return ok_; }
  bool is_err() const { return !ok_; }
  const RuntimeError &error() const { return err_; }
  T &value() { return value_; }
  const T &value() const { return value_; }
  T unwrap() && {
    if (!ok_) throw std::runtime_error(std::string(kind_name(err_.kind)) + ": " + err_.message);
    return std::move(value_);
  }

 private:
  bool ok_;
  T value_{};
  RuntimeError err_{};
};

template <>
class [[nodiscard]] Result<void> {
 public:
  Result() : ok_(true) {}
  Result(RuntimeError err) : ok_(false), err_(std::move(err)) {}
  bool is_ok() const { return ok_; }
  bool is_err() const { return !ok_; }
  const RuntimeError &error() const { return err_; }
  void unwrap() const {
    if (!ok_) throw std::runtime_error(std::string(kind_name(err_.kind)) + ": " + err_.message);
  }

 private:
  bool ok_;
  RuntimeError err_{};
};

namespace detail {
inline RuntimeError error_from(int code) {
  const char *msg = spissa_last_error();
  ErrorKind k = code == SPISSA_ERR_SHAPE                 ? ErrorKind::Shape
                : code == SPISSA_ERR_INVALID_TENSOR_DATA ? ErrorKind::InvalidTensorData
                : code == SPISSA_ERR_DEVICE              ? ErrorKind::Device
                                                         : ErrorKind::Argument;
  return RuntimeError{k, msg ? msg : ""};
}
inline Result<void> check(int code) {
  if (code == SPISSA_OK) return Result<void>();
  return Result<void>(error_from(code));
}
}  // namespace detail

// A borrowed slice (Rust &[T] / &mut [T]).
template <class T>
struct Slice {
  T *ptr = nullptr;
  size_t len = 0;
  Slice() = default;
  Slice(T *p, size_t n) : ptr(p), len(n) {}
  // Any contiguous container whose data() converts to T* (std::vector,
  // std::array, ...); temporaries bind to read-only slices for the call.
  template <class V, class = std::enable_if_t<std::is_convertible<decltype(std::declval<V &>().data()), T *>::value>>
  Slice(V &&v) : ptr(v.data()), len(v.size()) {}
  Slice sub(size_t from, size_t to) const { return Slice(ptr + from, to - from); }
  Slice sub(size_t from) const { return Slice(ptr + from, len - from); }
};

// rotary.rs:6-14
struct RotaryEmbeddingConfig {
  size_t seq_len;
  size_t num_heads;
  size_t head_dim;
  size_t rotary_dim;
  float base;
  size_t position_offset;

  spissa_rotary_config c() const {
    return spissa_rotary_config{seq_len, num_heads, head_dim, rotary_dim, base, position_offset};
  }
};

// rotary.rs:17-38
inline Result<size_t> gpt_neox_rotary_dim(size_t head_dim, float rotary_pct) {
  size_t out = 0;
  auto r = detail::check(spissa_gpt_neox_rotary_dim(head_dim, rotary_pct, &out));
  if (r.is_err()) return r.error();
  return out;
}

// rotary.rs:45-69
inline Result<void> apply_gpt_neox_rotary_inplace(Slice<float> q, Slice<float> k, const RotaryEmbeddingConfig &cfg) {
  const auto c = cfg.c();
  return detail::check(spissa_apply_gpt_neox_rotary_inplace(q.ptr, q.len, k.ptr, k.len, &c));
}

// rotary.rs:75-125; freq_scale = nullptr is Option::None.
inline Result<void> apply_llama_rotary_inplace(Slice<float> q, Slice<float> k, size_t q_heads, size_t k_heads,
                                               const RotaryEmbeddingConfig &cfg,
                                               const std::vector<float> *freq_scale = nullptr) {
  const auto c = cfg.c();
  return detail::check(spissa_apply_llama_rotary_inplace(q.ptr, q.len, k.ptr, k.len, q_heads, k_heads, &c,
                                                         freq_scale ? freq_scale->data() : nullptr,
                                                         freq_scale ? freq_scale->size() : 0));
}

// rotary.rs:137-186
inline Result<void> apply_gemma_rotary_inplace(Slice<float> q, Slice<float> k, size_t q_heads, size_t k_heads,
                                               const RotaryEmbeddingConfig &cfg, float position_divisor) {
  const auto c = cfg.c();
  return detail::check(
      spissa_apply_gemma_rotary_inplace(q.ptr, q.len, k.ptr, k.len, q_heads, k_heads, &c, position_divisor));
}

// rotary.rs:195-318: an append-only per-layer cache, resident in HBM.
// Move-only; clone() copies it (the Rust type is Clone).
class KvCache {
 public:
  // rotary.rs:206-224 (KvCache::new)
  static Result<KvCache> create(size_t num_heads, size_t head_dim, size_t max_seq_len) {
    spissa_kv_cache *h = nullptr;
    auto r = detail::check(spissa_kv_cache_new(num_heads, head_dim, max_seq_len, &h));
    if (r.is_err()) return r.error();
    return KvCache(h);
  }
  KvCache() = default;
  KvCache(KvCache &&o) noexcept : h_(o.h_) { o.h_ = nullptr; }
  KvCache &operator=(KvCache &&o) noexcept {
    if (this != &o) {
      reset();
      h_ = o.h_;
      o.h_ = nullptr;
    }
    return *this;
  }
  KvCache(const KvCache &) = delete;
  KvCache &operator=(const KvCache &) = delete;
  ~KvCache() { reset(); }

  Result<KvCache> clone() const {
    spissa_kv_cache *h = nullptr;
    auto r = detail::check(spissa_kv_cache_clone(h_, &h));
    if (r.is_err()) return r.error();
    return KvCache(h);
  }
  // rotary.rs:226-256
  Result<void> append(Slice<const float> keys, Slice<const float> values, size_t token_count) {
    return detail::check(spissa_kv_cache_append(h_, keys.ptr, keys.len, values.ptr, values.len, token_count));
  }
  void clear() { spissa_kv_cache_clear(h_); }                                                  // rotary.rs:258-262
  Result<void> truncate(size_t len) { return detail::check(spissa_kv_cache_truncate(h_, len)); }  // rotary.rs:264-278
  size_t resident_bytes() const { return spissa_kv_cache_resident_bytes(h_); }                  // rotary.rs:280-285
  size_t len() const { return spissa_kv_cache_len(h_); }
  bool is_empty() const { return spissa_kv_cache_is_empty(h_) != 0; }
  size_t max_seq_len() const { return spissa_kv_cache_max_seq_len(h_); }
  size_t num_heads() const { return spissa_kv_cache_num_heads(h_); }
  size_t head_dim() const { return spissa_kv_cache_head_dim(h_); }
  // rotary.rs:307-313: the cached rows [len, H, d], copied to the host.
  std::vector<float> keys() const { return read(&spissa_kv_cache_read_keys); }
  std::vector<float> values() const { return read(&spissa_kv_cache_read_values); }
  spissa_kv_cache *raw() const { return h_; }
  const float *device_keys() const { return spissa_kv_cache_device_keys(h_); }
  const float *device_values() const { return spissa_kv_cache_device_values(h_); }
  // Device tier: token_count rows [token_count, H, d] already on the device.
  Result<void> append_device(const float *d_keys, const float *d_values, size_t token_count) {
    return detail::check(spissa_kv_cache_append_device(h_, d_keys, d_values, token_count));
  }

 private:
  friend class Session;
  explicit KvCache(spissa_kv_cache *h) : h_(h) {}
  void reset() {
    if (h_) spissa_kv_cache_free(h_);
    h_ = nullptr;
  }
  std::vector<float> read(int (*fn)(const spissa_kv_cache *, float *, size_t)) const {
    std::vector<float> out(len() * num_heads() * head_dim());
    if (!out.empty() && fn(h_, out.data(), out.size()) != SPISSA_OK)
      throw std::runtime_error(std::string("reading the KV cache failed: ") + spissa_last_error());
    return out;
  }
  spissa_kv_cache *h_ = nullptr;
};

// rotary.rs:320-327, plus the sliding-window extension (0 = none).
struct KvAttentionConfig {
  size_t query_len;
  size_t num_heads;
  size_t kv_heads;
  size_t head_dim;
  bool causal;
  size_t window = 0;

  spissa_kv_attention_config c() const {
    return spissa_kv_attention_config{query_len, num_heads, kv_heads, head_dim, causal ? 1 : 0, window};
  }
};

// rotary.rs:335-415; cache = nullptr is Option::None.
inline Result<std::vector<float>> scaled_dot_product_attention_with_cache(Slice<const float> q,
                                                                          Slice<const float> current_k,
                                                                          Slice<const float> current_v,
                                                                          const KvCache *cache,
                                                                          const KvAttentionConfig &config) {
  std::vector<float> out(config.query_len * config.num_heads * config.head_dim);
  const auto c = config.c();
  auto r = detail::check(spissa_scaled_dot_product_attention_with_cache(
      q.ptr, q.len, current_k.ptr, current_k.len, current_v.ptr, current_v.len, cache ? cache->raw() : nullptr, &c,
      out.data(), out.size()));
  if (r.is_err()) return r.error();
  return out;
}

namespace ops {
// ops.rs:159-179
inline Result<std::vector<float>> rms_norm(Slice<const float> x, Slice<const float> weight, size_t rows, size_t cols,
                                           float eps) {
  std::vector<float> out(x.len);
  auto r = detail::check(spissa_rms_norm(x.ptr, x.len, weight.ptr, weight.len, rows, cols, eps, out.data(), out.size()));
  if (r.is_err()) return r.error();
  return out;
}
// ops.rs:237-291
inline Result<std::vector<float>> scaled_dot_product_attention(Slice<const float> q, Slice<const float> k,
                                                               Slice<const float> v, size_t seq_len, size_t num_heads,
                                                               size_t head_dim, bool causal) {
  std::vector<float> out(q.len);
  auto r = detail::check(spissa_scaled_dot_product_attention(q.ptr, q.len, k.ptr, k.len, v.ptr, v.len, seq_len,
                                                             num_heads, head_dim, causal ? 1 : 0, out.data(),
                                                             out.size()));
  if (r.is_err()) return r.error();
  return out;
}
}  // namespace ops

// models/gemma/model.rs:46-51
inline bool is_global_layer(size_t layer_idx, size_t sliding_window_pattern) {
  return spissa_is_global_layer(layer_idx, sliding_window_pattern) != 0;
}

// ---- linear projections (streaming/linear.rs:269-576) ----

enum class DType { F32 = SPISSA_DTYPE_F32, F16 = SPISSA_DTYPE_F16, Bf16 = SPISSA_DTYPE_BF16 };

// streaming/mod.rs:511-516
struct StreamingLinearConfig {
  size_t batch;
  size_t in_features;
  size_t out_features;
  spissa_linear_config c() const { return spissa_linear_config{batch, in_features, out_features}; }
};

// streaming/mod.rs:518-526. tile_elements bounds the reference's f32 CPU
// scratch; the device path has none, so it is only validated (> 0).
struct StreamingTileLinearConfig {
  StreamingLinearConfig linear;
  size_t tile_elements;
};

class Session;

// A [out_features, in_features] row-major weight resident in HBM, uploaded
// from its raw little-endian element bytes. Free it before its session.
class LinearWeight {
 public:
  // session = nullptr: the calling thread's default session.
  static Result<LinearWeight> create(DType dtype, size_t out_features, size_t in_features, const void *data,
                                     size_t data_bytes, const Session *session = nullptr);
  LinearWeight() = default;
  LinearWeight(LinearWeight &&o) noexcept
      : w_(o.w_), dtype_(o.dtype_), out_features_(o.out_features_), in_features_(o.in_features_) {
    o.w_ = nullptr;
  }
  LinearWeight &operator=(LinearWeight &&o) noexcept {
    if (this != &o) {
      if (w_) spissa_linear_weight_free(w_);
      w_ = o.w_;
      dtype_ = o.dtype_;
      out_features_ = o.out_features_;
      in_features_ = o.in_features_;
      o.w_ = nullptr;
    }
    return *this;
  }
  LinearWeight(const LinearWeight &) = delete;
  LinearWeight &operator=(const LinearWeight &) = delete;
  ~LinearWeight() {
    if (w_) spissa_linear_weight_free(w_);
  }
  spissa_linear_weight *raw() const { return w_; }
  DType dtype() const { return dtype_; }
  size_t out_features() const { return out_features_; }
  size_t in_features() const { return in_features_; }

 private:
  LinearWeight(spissa_linear_weight *w, DType dtype, size_t out_features, size_t in_features)
      : w_(w), dtype_(dtype), out_features_(out_features), in_features_(in_features) {}
  spissa_linear_weight *w_ = nullptr;
  DType dtype_ = DType::F32;
  size_t out_features_ = 0, in_features_ = 0;
};

// Resident weights by tensor name: the role of lazy.rs's LazySpissaModel.
class LinearModel {
 public:
  void add(const std::string &name, LinearWeight w) { w_[name] = std::move(w); }
  // lazy.rs:357-361
  Result<const LinearWeight *> tensor(const std::string &name) const {
    auto it = w_.find(name);
    if (it == w_.end()) return RuntimeError{ErrorKind::MissingTensor, name};
    return &it->second;
  }

 private:
  std::map<std::string, LinearWeight> w_;
};

// input[batch, in] x W^T + bias on the GPU (ops.rs:62-105 arithmetic in f32);
// bias = nullptr is Option::None. Shape errors as streaming/validation.rs:225-289.
inline Result<std::vector<float>> linear(const LinearWeight &w, Slice<const float> input,
                                         const std::vector<float> *bias, const StreamingLinearConfig &config) {
  std::vector<float> out(config.batch * config.out_features);
  const auto c = config.c();
  auto r = detail::check(spissa_linear(w.raw(), input.ptr, input.len, bias ? bias->data() : nullptr,
                                       bias ? bias->size() : 0, &c, out.data(), out.size()));
  if (r.is_err()) return r.error();
  return out;
}

// streaming/linear.rs:269-576 with the weight already resident.
inline Result<std::vector<float>> streaming_tile_linear_from_model(const LinearModel &model,
                                                                   const std::string &weight_name,
                                                                   Slice<const float> input,
                                                                   const std::vector<float> *bias,
                                                                   const StreamingTileLinearConfig &config) {
  if (config.tile_elements == 0)  // streaming/validation.rs:249-256
    return RuntimeError{ErrorKind::Shape, "tile_elements must be greater than zero"};
  auto w = model.tensor(weight_name);
  if (w.is_err()) return w.error();
  return linear(*w.value(), input, bias, config.linear);
}

// ---- LM head and greedy sampling (streaming/mod.rs:186-287, ops.rs:309-348) ----

namespace detail {
inline Result<std::vector<float>> lm_head(Slice<const float> last_hidden, const LinearWeight &table,
                                          size_t vocab_size, size_t hidden, DType want) {
  if (table.dtype() != want)
    return RuntimeError{ErrorKind::InvalidTensorData, "LM head table dtype does not match this variant"};
  if (table.out_features() != vocab_size || table.in_features() != hidden)
    return RuntimeError{ErrorKind::Shape, "LM head table shape does not match vocab_size x hidden"};
  std::vector<float> logits(vocab_size);
  auto r = detail::check(spissa_lm_head_logits(table.raw(), last_hidden.ptr, last_hidden.len, logits.data(),
                                               logits.size()));
  if (r.is_err()) return r.error();
  return logits;
}
inline int64_t excluded_arg(std::optional<size_t> e) {
  // an index past INT64_MAX is past any logits buffer: plain sample_argmax either way
  return e && *e <= static_cast<size_t>(INT64_MAX) ? static_cast<int64_t>(*e) : -1;
}
}  // namespace detail

// streaming/mod.rs:186-221: logits[v] = sum_h last_hidden[h] * table[v, h] over a
// resident f32 table [vocab_size, hidden] (the tied embedding).
inline Result<std::vector<float>> lm_head_logits_parallel(Slice<const float> last_hidden, const LinearWeight &table,
                                                          size_t vocab_size, size_t hidden) {
  return detail::lm_head(last_hidden, table, vocab_size, hidden, DType::F32);
}
// streaming/mod.rs:238-272, resident bf16 table.
inline Result<std::vector<float>> lm_head_logits_parallel_bf16(Slice<const float> last_hidden,
                                                               const LinearWeight &table, size_t vocab_size,
                                                               size_t hidden) {
  return detail::lm_head(last_hidden, table, vocab_size, hidden, DType::Bf16);
}

// ops.rs:326-348 (std::nullopt: ops.rs:309-324 sample_argmax), on the calling
// thread's default session.
inline Result<size_t> sample_argmax_excluding(Slice<const float> logits, std::optional<size_t> excluded_token) {
  spissa_session *s = nullptr;
  auto r = detail::check(spissa_default_session(&s));
  if (r.is_err()) return r.error();
  size_t token = 0;
  r = detail::check(spissa_sample_argmax(s, logits.ptr, logits.len, detail::excluded_arg(excluded_token), &token));
  if (r.is_err()) return r.error();
  return token;
}
inline Result<size_t> sample_argmax(Slice<const float> logits) { return sample_argmax_excluding(logits, std::nullopt); }

// ---- device tier (no reference counterpart): device pointers, one stream ----

enum class RopeKind { Llama = SPISSA_ROPE_LLAMA, Gemma = SPISSA_ROPE_GEMMA, Neox = SPISSA_ROPE_NEOX };

// A resident cos/sin table for positions [0, max_positions), bit-identical to
// the host formulas of rotary.rs:454-465 (Llama, Neox) and 168,188-193 (Gemma).
class RopeTable {
 public:
  RopeTable() = default;
  RopeTable(RopeTable &&o) noexcept : t_(o.t_) { o.t_ = nullptr; }
  RopeTable &operator=(RopeTable &&o) noexcept {
    if (this != &o) {
      if (t_) spissa_rope_table_free(t_);
      t_ = o.t_;
      o.t_ = nullptr;
    }
    return *this;
  }
  RopeTable(const RopeTable &) = delete;
  RopeTable &operator=(const RopeTable &) = delete;
  ~RopeTable() {
    if (t_) spissa_rope_table_free(t_);
  }
  spissa_rope_table *raw() const { return t_; }

 private:
  friend class Session;
  explicit RopeTable(spissa_rope_table *t) : t_(t) {}
  spissa_rope_table *t_ = nullptr;
};

// One layer's attention sublayer (models/gemma/generate.rs:178-312,
// models/llama/generate.rs:200-450): weights, norm multipliers (device
// pointers, nullptr: that norm is absent), the layer's rope table.
struct AttentionLayer {
  size_t hidden, q_heads, kv_heads, head_dim;
  const LinearWeight *q_weight, *k_weight, *v_weight, *o_weight;
  const float *d_input_norm = nullptr;
  const float *d_q_norm = nullptr;
  const float *d_k_norm = nullptr;
  const float *d_post_norm = nullptr;
  float eps = 1e-6f;
  const RopeTable *rope = nullptr;
  float q_prescale = 1.0f;
  bool causal = true;
  size_t window = 0;

  spissa_attention_layer c() const {
    return spissa_attention_layer{hidden, q_heads, kv_heads, head_dim, q_weight ? q_weight->raw() : nullptr,
                                  k_weight ? k_weight->raw() : nullptr, v_weight ? v_weight->raw() : nullptr,
                                  o_weight ? o_weight->raw() : nullptr, d_input_norm, d_q_norm, d_k_norm,
                                  d_post_norm, eps, rope ? rope->raw() : nullptr, q_prescale, causal ? 1 : 0,
                                  window};
  }
};

// One device and one HIP stream. Calls are asynchronous on that stream;
// sync() waits and reports device-side errors.
class Session {
 public:
  // stream = nullptr creates an owned stream; otherwise the caller's HIP stream is used.
  static Result<Session> create(int device = 0, void *stream = nullptr) {
    spissa_session *s = nullptr;
    auto r = detail::check(spissa_session_create(device, stream, &s));
    if (r.is_err()) return r.error();
    return Session(s);
  }
  Session() = default;
  Session(Session &&o) noexcept : s_(o.s_) { o.s_ = nullptr; }
  Session &operator=(Session &&o) noexcept {
    if (this != &o) {
      if (s_) spissa_session_destroy(s_);
      s_ = o.s_;
      o.s_ = nullptr;
    }
    return *this;
  }
  Session(const Session &) = delete;
  Session &operator=(const Session &) = delete;
  ~Session() {
    if (s_) spissa_session_destroy(s_);
  }
  spissa_session *raw() const { return s_; }
  void *stream() const { return spissa_session_stream(s_); }
  int device() const { return spissa_session_device(s_); }
  // Waits for the session's work; reports device-side errors (an invalid
  // softmax denominator is InvalidTensorData, rotary.rs:560-564).
  Result<void> sync() const { return detail::check(spissa_session_sync(s_)); }
  Result<void> set_prefill_precision(int precision) const {
    return detail::check(spissa_session_set_prefill_precision(s_, precision));
  }

  // KvCache::new bound to this session's device and stream.
  Result<KvCache> kv_cache(size_t num_heads, size_t head_dim, size_t max_seq_len) const {
    spissa_kv_cache *h = nullptr;
    auto r = detail::check(spissa_kv_cache_new_in(s_, num_heads, head_dim, max_seq_len, &h));
    if (r.is_err()) return r.error();
    return KvCache(h);
  }
  // freq_scale: Llama per-pair scales (nullptr = None); position_divisor: Gemma only.
  Result<RopeTable> rope_table(RopeKind kind, size_t rotary_dim, float base, size_t max_positions,
                               float position_divisor = 1.0f,
                               const std::vector<float> *freq_scale = nullptr) const {
    spissa_rope_table *t = nullptr;
    auto r = detail::check(spissa_rope_table_new(s_, static_cast<int>(kind), rotary_dim, base, position_divisor,
                                                 freq_scale ? freq_scale->data() : nullptr,
                                                 freq_scale ? freq_scale->size() : 0, max_positions, &t));
    if (r.is_err()) return r.error();
    return RopeTable(t);
  }
  Result<void> rope(const RopeTable &t, float *d_q, float *d_k, size_t seq_len, size_t q_heads, size_t k_heads,
                    size_t head_dim, size_t position_offset) const {
    return detail::check(
        spissa_rope_apply_device(s_, t.raw(), d_q, d_k, seq_len, q_heads, k_heads, head_dim, position_offset));
  }
  Result<void> rms_norm(const float *d_x, const float *d_weight, size_t rows, size_t cols, float eps,
                        float *d_out) const {
    return detail::check(spissa_rms_norm_device(s_, d_x, d_weight, rows, cols, eps, d_out));
  }
  // models/gemma/generate.rs:230-278: QK-norm, Gemma RoPE, q prescale, in place.
  Result<void> gemma_qk_prologue(const RopeTable &t, float *d_q, float *d_k, size_t seq_len, size_t q_heads,
                                 size_t kv_heads, size_t head_dim, const float *d_q_norm, const float *d_k_norm,
                                 float eps, size_t position_offset, float q_prescale) const {
    return detail::check(spissa_gemma_qk_prologue_device(s_, t.raw(), d_q, d_k, seq_len, q_heads, kv_heads, head_dim,
                                                         d_q_norm, d_k_norm, eps, position_offset, q_prescale));
  }
  // rotary.rs:335-415 on device buffers.
  Result<void> attention(const float *d_q, const float *d_k, const float *d_v, const KvCache *cache,
                         const KvAttentionConfig &cfg, float *d_out) const {
    const auto c = cfg.c();
    return detail::check(spissa_attention_device(s_, d_q, d_k, d_v, cache ? cache->raw() : nullptr, &c, d_out));
  }
  // Single-token attention of `caches.size()` sequences in one launch.
  Result<void> attention_decode_batch(const float *d_q, const float *d_k, const float *d_v,
                                      const std::vector<const KvCache *> &caches, const KvAttentionConfig &cfg,
                                      float *d_out) const {
    std::vector<const spissa_kv_cache *> raw(caches.size());
    for (size_t i = 0; i < caches.size(); ++i) raw[i] = caches[i] ? caches[i]->raw() : nullptr;
    const auto c = cfg.c();
    return detail::check(
        spissa_attention_decode_batch_device(s_, d_q, d_k, d_v, raw.data(), raw.size(), &c, d_out));
  }
  // The attention sublayer of one layer: d_x [seq_len, hidden] -> d_out; RoPE
  // positions continue the cache, whose rows receive the rotated k and v.
  Result<void> attention_sublayer(const AttentionLayer &layer, const float *d_x, size_t seq_len, KvCache *cache,
                                  float *d_out) const {
    const auto c = layer.c();
    return detail::check(
        spissa_attention_sublayer_device(s_, &c, d_x, seq_len, cache ? cache->raw() : nullptr, d_out));
  }
  // out[batch, out] = x[batch, in] x W^T + bias on device buffers (d_bias may be null).
  Result<void> linear(const LinearWeight &w, const float *d_x, const float *d_bias, size_t batch,
                      float *d_out) const {
    return detail::check(spissa_linear_device(s_, w.raw(), d_x, d_bias, batch, d_out));
  }
  Result<LinearWeight> linear_weight(DType dtype, size_t out_features, size_t in_features, const void *data,
                                     size_t data_bytes) const {
    return LinearWeight::create(dtype, out_features, in_features, data, data_bytes, this);
  }
  // d_token[0] = sample_argmax_excluding(d_logits[0..n), excluded) on the device.
  Result<void> argmax(const float *d_logits, size_t n, int32_t *d_token,
                      std::optional<size_t> excluded = std::nullopt) const {
    return detail::check(spissa_argmax_device(s_, d_logits, n, detail::excluded_arg(excluded), d_token));
  }
  // The greedy decode tail: d_logits = table x d_hidden, then (d_token set) its argmax.
  Result<void> lm_head(const LinearWeight &table, const float *d_hidden, float *d_logits, int32_t *d_token = nullptr,
                       std::optional<size_t> excluded = std::nullopt) const {
    return detail::check(
        spissa_lm_head_device(s_, table.raw(), d_hidden, detail::excluded_arg(excluded), d_logits, d_token));
  }
  // RoPE + attention + append of one decode step of one layer (table = nullptr: no RoPE).
  Result<void> decode_step(const RopeTable *table, const float *d_q, const float *d_k, const float *d_v,
                           const std::vector<KvCache *> &caches, const KvAttentionConfig &cfg, float *d_out) const {
    std::vector<spissa_kv_cache *> raw(caches.size());
    for (size_t i = 0; i < caches.size(); ++i) raw[i] = caches[i] ? caches[i]->raw() : nullptr;
    const auto c = cfg.c();
    return detail::check(spissa_decode_step_device(s_, table ? table->raw() : nullptr, d_q, d_k, d_v, raw.data(),
                                                   raw.size(), &c, d_out));
  }

 private:
  explicit Session(spissa_session *s) : s_(s) {}
  spissa_session *s_ = nullptr;
};

inline Result<LinearWeight> LinearWeight::create(DType dtype, size_t out_features, size_t in_features,
                                                 const void *data, size_t data_bytes, const Session *session) {
  spissa_session *s = nullptr;
  if (session) {
    s = session->raw();
  } else {
    auto r = detail::check(spissa_default_session(&s));
    if (r.is_err()) return r.error();
  }
  spissa_linear_weight *w = nullptr;
  auto r = detail::check(
      spissa_linear_weight_new(s, static_cast<int>(dtype), out_features, in_features, data, data_bytes, &w));
  if (r.is_err()) return r.error();
  return LinearWeight(w, dtype, out_features, in_features);
}

}  // namespace spissa
