/*
 * spissa_oracle.h -- CPU restatement of the Spissa runtime's attention path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * path in spissa_amd/: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only to check or time the reference
 * algorithm. The product never links it and never falls back to it.
 *
 * Each function restates one function of the Rust reference
 * (crates/spissa-runtime/src/rotary.rs, crates/spissa-runtime/src/ops.rs,
 * crates/spissa-runtime/src/models/gemma/{generate,model}.rs) in plain C with
 * the same loop order and the same f32 operation order. It is compiled with
 * -fno-fast-math -ffp-contract=off against glibc libm (powf, cosf, sinf, expf,
 * sqrtf), which is what Rust's f32 methods lower to on x86_64-linux-gnu.
 *
 * Status codes mirror RuntimeError variants (crates/spissa-runtime/src/error.rs:6-54):
 *   0 = Ok, 1 = Shape, 2 = InvalidTensorData.
 * Where the Rust reference would panic (out-of-range slice index) the oracle
 * returns Shape instead; no such case is reachable from valid callers.
 */
#ifndef SPISSA_ORACLE_H
#define SPISSA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_OK = 0, OR_SHAPE = 1, OR_INVALID = 2 };

/* rotary.rs:6-14 */
typedef struct {
    size_t seq_len;
    size_t num_heads;
    size_t head_dim;
    size_t rotary_dim;
    float base;
    size_t position_offset;
} or_rotary_config;

/* rotary.rs:320-327, plus the sliding-window extension (window = 0: none). */
typedef struct {
    size_t query_len;
    size_t num_heads;
    size_t kv_heads;
    size_t head_dim;
    int causal;
    size_t window;
} or_kv_attention_config;

/* rotary.rs:195-203 */
typedef struct {
    size_t num_heads;
    size_t head_dim;
    size_t max_seq_len;
    size_t len;
    float *keys;   /* capacity max_seq_len * num_heads * head_dim */
    float *values;
} or_kv_cache;

const char *or_last_error(void);

int or_gpt_neox_rotary_dim(size_t head_dim, float rotary_pct, size_t *out);
int or_apply_gpt_neox_rotary_inplace(float *q, size_t q_len, float *k, size_t k_len,
                                     const or_rotary_config *cfg);
int or_apply_llama_rotary_inplace(float *q, size_t q_len, float *k, size_t k_len,
                                  size_t q_heads, size_t k_heads, const or_rotary_config *cfg,
                                  const float *freq_scale, size_t freq_scale_len);
int or_apply_gemma_rotary_inplace(float *q, size_t q_len, float *k, size_t k_len,
                                  size_t q_heads, size_t k_heads, const or_rotary_config *cfg,
                                  float position_divisor);
/* Per-(position, pair) cos/sin exactly as rotary.rs computes them, for tables. */
void or_llama_cos_sin(size_t absolute_pos, size_t pair, size_t rotary_dim, float base,
                      float freq_scale, float *cos_out, float *sin_out);
void or_gemma_cos_sin(size_t absolute_pos, size_t pair, size_t rotary_dim, float base,
                      float position_divisor, float *cos_out, float *sin_out);

or_kv_cache *or_kv_new(size_t num_heads, size_t head_dim, size_t max_seq_len, int *status);
void or_kv_free(or_kv_cache *c);
int or_kv_append(or_kv_cache *c, const float *keys, size_t keys_len, const float *values,
                 size_t values_len, size_t token_count);
void or_kv_clear(or_kv_cache *c);
int or_kv_truncate(or_kv_cache *c, size_t len);
size_t or_kv_resident_bytes(const or_kv_cache *c);
size_t or_kv_len(const or_kv_cache *c);
const float *or_kv_keys(const or_kv_cache *c);
const float *or_kv_values(const or_kv_cache *c);

int or_sdpa_with_cache(const float *q, size_t q_len, const float *cur_k, size_t k_len,
                       const float *cur_v, size_t v_len, const or_kv_cache *cache,
                       const or_kv_attention_config *cfg, float *out, size_t out_len);

int or_rms_norm(const float *x, size_t x_len, const float *w, size_t w_len, size_t rows,
                size_t cols, float eps, float *out);
int or_softmax_rows(const float *logits, size_t len, size_t rows, size_t cols, float *out);
int or_scaled_dot_product_attention(const float *q, const float *k, const float *v, size_t len,
                                    size_t seq_len, size_t num_heads, size_t head_dim,
                                    int causal, float *out);

int or_is_global_layer(size_t layer_idx, size_t sliding_window_pattern);

/* Weight element types (spissa_container::DType Fp32, Fp16, Bf16). */
enum { OR_DTYPE_F32 = 0, OR_DTYPE_F16 = 1, OR_DTYPE_BF16 = 2 };
/* tensor.rs:217-221 bf16_to_f32 */
float or_bf16_to_f32(uint16_t bits);
/* tensor.rs:166-215 fp16_to_f32 (exact binary16 decode) */
float or_fp16_to_f32(uint16_t bits);
/* streaming/mod.rs:366-374 f32_to_bf16_rne */
uint16_t or_f32_to_bf16_rne(float x);
/* ops.rs:62-105 linear over the weight decoded to f32 (tensor.rs:84-100
 * decode_to_f32): out[b][o] = bias[o] + sum_i input[b][i] * w[o][i], the sum
 * running from the bias in index order with each product rounded first. This
 * is also the order of the reference's exact batch-1 row-block loop
 * (streaming/kernels_raw16.rs:640-672). weight_elems counts elements. */
int or_linear(const float *input, size_t input_len, const void *weight, int dtype, size_t weight_elems,
              const float *bias, size_t bias_len, size_t batch, size_t in_features,
              size_t out_features, float *out);
/* streaming/mod.rs:223-236 lm_head_logits_rows (f32 table, dtype OR_DTYPE_F32)
 * and streaming/mod.rs:274-287 with the scalar row dot of streaming/mod.rs:309-319
 * (bf16 table, OR_DTYPE_BF16): logits[v] = sum_h last_hidden[h] * table[v][h],
 * from 0.0 in index order with each product rounded. The parallel entry
 * points (streaming/mod.rs:186-221, 238-272) only split the rows over
 * threads, so they equal this serial loop bit for bit. */
int or_lm_head_logits(const float *last_hidden, size_t hidden_len, const void *table, int dtype,
                      size_t vocab_size, size_t hidden, float *logits);
/* ops.rs:309-324 sample_argmax */
int or_sample_argmax(const float *logits, size_t n, size_t *out);
/* ops.rs:326-348 sample_argmax_excluding; has_excluded == 0 is Option::None */
int or_sample_argmax_excluding(const float *logits, size_t n, int has_excluded, size_t excluded,
                               size_t *out);
int or_gemma_qk_prologue(float *q, size_t q_len, float *k, size_t k_len, size_t seq_len,
                         size_t q_heads, size_t kv_heads, size_t head_dim, const float *q_norm,
                         const float *k_norm, float eps, float rope_base,
                         float position_divisor, size_t position_offset,
                         float query_pre_attn_scalar);

/* Harness helper (not part of the reference): runs or_sdpa_with_cache over
 * `units` independent (cache, q, k, v) sets on `threads` POSIX threads. */
int or_sdpa_many_threads(size_t units, const float *const *q, const float *const *k,
                         const float *const *v, const or_kv_cache *const *caches,
                         const or_kv_attention_config *cfg, float *const *out, int threads);

#ifdef __cplusplus
}
#endif
#endif
