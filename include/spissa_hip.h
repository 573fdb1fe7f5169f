/*
 * spissa_hip.h -- C ABI of the MI355X (gfx950) attention path for the Spissa
 * runtime: RoPE, the per-layer KV cache, cached SDPA (decode and causal GQA
 * prefill), the Gemma 3 QK-norm, the linear projections either side, and
 * the LM head with greedy sampling after the last layer.
 *
 * Every symbol here replaces one Rust item of crates/spissa-runtime; the
 * citation next to each declaration names it (paths relative to the
 * reference repository root). The ABI is plain C: pointers, sizes and status
 * codes, no C++ or torch types.
 *
 * Two kinds of entry points:
 *   - drop-in (no suffix): host pointers, exactly the Rust argument meaning and
 *     error behaviour; synchronous; results are host-visible on return;
 *   - device (`_device` suffix): device pointers, asynchronous on the
 *     session's HIP stream; device-side errors (invalid softmax denominator)
 *     are reported by the next spissa_session_sync().
 *
 * Status codes map onto RuntimeError variants
 * (crates/spissa-runtime/src/error.rs:6-54). Validation always happens before
 * any mutation, as in the reference. No call aborts or lets an exception out.
 */
#ifndef SPISSA_HIP_H
#define SPISSA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    SPISSA_OK = 0,
    SPISSA_ERR_SHAPE = 1,               /* RuntimeError::Shape (error.rs:12) */
    SPISSA_ERR_INVALID_TENSOR_DATA = 2, /* RuntimeError::InvalidTensorData (error.rs:24) */
    SPISSA_ERR_DEVICE = 3,              /* HIP runtime failure; no reference counterpart */
    SPISSA_ERR_ARGUMENT = 4             /* null handle or pointer; no reference counterpart */
} spissa_status;

/* Thread-local message of the last failing call on this thread. */
const char *spissa_last_error(void);
const char *spissa_version(void);

/* ------------------------------------------------------------------------ */
/* Sessions: one device, one HIP stream, one growable device workspace.     */
/* The reference has no counterpart (it is synchronous, single-threaded:     */
/* crates/spissa-runtime/src/rotary.rs:335-415); a session is the device     */
/* context the drop-in calls run in. Drop-in calls use the calling thread's  */
/* default session (current HIP device at first use).                       */
/* ------------------------------------------------------------------------ */
typedef struct spissa_session spissa_session;

/* stream: an existing hipStream_t to run on (not owned), or NULL to create one. */
int spissa_session_create(int device, void *stream, spissa_session **out);
/* Releases the caller's session; its memory goes when the last cache and
 * weight created on it have been freed too (they hold references). */
void spissa_session_destroy(spissa_session *s);
int spissa_default_session(spissa_session **out);
/* Wait for all work of the session; returns INVALID_TENSOR_DATA if a device
 * kernel saw an invalid softmax denominator since the last sync. */
int spissa_session_sync(spissa_session *s);
void *spissa_session_stream(spissa_session *s);
int spissa_session_device(const spissa_session *s);

/* ------------------------------------------------------------------------ */
/* KV cache: rotary.rs:195-318 (KvCache). Device-resident, appended in place. */
/* Layout of keys and values in HBM: [max_seq_len, num_heads, head_dim] f32,  */
/* row-major, so the first len rows are byte-identical to KvCache::keys().    */
/* ------------------------------------------------------------------------ */
typedef struct spissa_kv_cache spissa_kv_cache;

/* rotary.rs:206-224 KvCache::new (on the calling thread's default session). */
int spissa_kv_cache_new(size_t num_heads, size_t head_dim, size_t max_seq_len,
                        spissa_kv_cache **out);
/* Same, bound to an explicit session. */
int spissa_kv_cache_new_in(spissa_session *s, size_t num_heads, size_t head_dim,
                           size_t max_seq_len, spissa_kv_cache **out);
/* Drop impl of KvCache. */
void spissa_kv_cache_free(spissa_kv_cache *c);
/* #[derive(Clone)] on KvCache (rotary.rs:195). */
int spissa_kv_cache_clone(const spissa_kv_cache *c, spissa_kv_cache **out);
/* rotary.rs:226-256 KvCache::append (host buffers; validates before mutating). */
int spissa_kv_cache_append(spissa_kv_cache *c, const float *keys, size_t keys_len,
                           const float *values, size_t values_len, size_t token_count);
/* Same contract with device buffers of token_count*num_heads*head_dim floats. */
int spissa_kv_cache_append_device(spissa_kv_cache *c, const float *d_keys,
                                  const float *d_values, size_t token_count);
/* rotary.rs:258-262 KvCache::clear */
void spissa_kv_cache_clear(spissa_kv_cache *c);
/* rotary.rs:264-278 KvCache::truncate */
int spissa_kv_cache_truncate(spissa_kv_cache *c, size_t len);
/* rotary.rs:280-305 accessors */
size_t spissa_kv_cache_len(const spissa_kv_cache *c);
int spissa_kv_cache_is_empty(const spissa_kv_cache *c);
size_t spissa_kv_cache_max_seq_len(const spissa_kv_cache *c);
size_t spissa_kv_cache_num_heads(const spissa_kv_cache *c);
size_t spissa_kv_cache_head_dim(const spissa_kv_cache *c);
size_t spissa_kv_cache_resident_bytes(const spissa_kv_cache *c);
/* rotary.rs:307-313 keys()/values(): copy len*num_heads*head_dim floats to host. */
int spissa_kv_cache_read_keys(const spissa_kv_cache *c, float *dst, size_t dst_len);
int spissa_kv_cache_read_values(const spissa_kv_cache *c, float *dst, size_t dst_len);
/* Device base pointers of the resident buffers (fast path, no reference counterpart). */
const float *spissa_kv_cache_device_keys(const spissa_kv_cache *c);
const float *spissa_kv_cache_device_values(const spissa_kv_cache *c);

/* ------------------------------------------------------------------------ */
/* RoPE: rotary.rs:6-193                                                    */
/* ------------------------------------------------------------------------ */

/* rotary.rs:6-14 RotaryEmbeddingConfig */
typedef struct {
    size_t seq_len;
    size_t num_heads;
    size_t head_dim;
    size_t rotary_dim;
    float base;
    size_t position_offset;
} spissa_rotary_config;

/* rotary.rs:17-38 gpt_neox_rotary_dim */
int spissa_gpt_neox_rotary_dim(size_t head_dim, float rotary_pct, size_t *out);
/* rotary.rs:45-69 apply_gpt_neox_rotary_inplace */
int spissa_apply_gpt_neox_rotary_inplace(float *q, size_t q_len, float *k, size_t k_len,
                                         const spissa_rotary_config *cfg);
/* rotary.rs:75-125 apply_llama_rotary_inplace; freq_scale may be NULL (Option::None). */
int spissa_apply_llama_rotary_inplace(float *q, size_t q_len, float *k, size_t k_len,
                                      size_t q_heads, size_t k_heads,
                                      const spissa_rotary_config *cfg, const float *freq_scale,
                                      size_t freq_scale_len);
/* rotary.rs:137-186 apply_gemma_rotary_inplace */
int spissa_apply_gemma_rotary_inplace(float *q, size_t q_len, float *k, size_t k_len,
                                      size_t q_heads, size_t k_heads,
                                      const spissa_rotary_config *cfg, float position_divisor);

/* Resident cos/sin table for positions [0, max_positions): computed once on
 * the host with the exact per-(position, pair) formulas of rotary.rs:454-465
 * (LLAMA, NEOX) or rotary.rs:168,188-193 (GEMMA) and applied on the device,
 * so device RoPE is bit-identical to the drop-in call. */
typedef enum { SPISSA_ROPE_LLAMA = 0, SPISSA_ROPE_GEMMA = 1, SPISSA_ROPE_NEOX = 2 } spissa_rope_kind;
typedef struct spissa_rope_table spissa_rope_table;
int spissa_rope_table_new(spissa_session *s, int kind, size_t rotary_dim, float base,
                          float position_divisor, const float *freq_scale, size_t freq_scale_len,
                          size_t max_positions, spissa_rope_table **out);
void spissa_rope_table_free(spissa_rope_table *t);
/* Device RoPE on q [seq_len, q_heads, head_dim] and k [seq_len, k_heads, head_dim]
 * at absolute positions position_offset + s. */
int spissa_rope_apply_device(spissa_session *s, const spissa_rope_table *t, float *d_q,
                             float *d_k, size_t seq_len, size_t q_heads, size_t k_heads,
                             size_t head_dim, size_t position_offset);

/* ------------------------------------------------------------------------ */
/* RMSNorm / Gemma QK-norm                                                  */
/* ------------------------------------------------------------------------ */

/* ops.rs:159-179 rms_norm (bit-identical: sequential sum of squares per row). */
int spissa_rms_norm(const float *x, size_t x_len, const float *weight, size_t weight_len,
                    size_t rows, size_t cols, float eps, float *out, size_t out_len);
int spissa_rms_norm_device(spissa_session *s, const float *d_x, const float *d_weight,
                           size_t rows, size_t cols, float eps, float *d_out);
/* models/gemma/model.rs:46-51 is_global_layer */
int spissa_is_global_layer(size_t layer_idx, size_t sliding_window_pattern);
/* models/gemma/generate.rs:230-278 fused on the device: QK-norm of q and k
 * rows, Gemma RoPE from `t` (built with the layer's base and divisor), then
 * q *= q_prescale, with q_prescale = (1/sqrt(query_pre_attn_scalar))*sqrt(head_dim)
 * as models/gemma/generate.rs:275 computes it. In place. */
int spissa_gemma_qk_prologue_device(spissa_session *s, const spissa_rope_table *t, float *d_q,
                                    float *d_k, size_t seq_len, size_t q_heads, size_t kv_heads,
                                    size_t head_dim, const float *d_q_norm,
                                    const float *d_k_norm, float eps, size_t position_offset,
                                    float q_prescale);

/* ------------------------------------------------------------------------ */
/* Attention                                                                */
/* ------------------------------------------------------------------------ */

/* rotary.rs:320-327 KvAttentionConfig, extended with a sliding window:
 * window = 0 is the reference (no window); window = W > 0 additionally masks
 * keys j with j + W <= i for a query at absolute position i (i-W < j <= i). */
typedef struct {
    size_t query_len;
    size_t num_heads;
    size_t kv_heads;
    size_t head_dim;
    int causal;
    size_t window;
} spissa_kv_attention_config;

/* rotary.rs:335-415 scaled_dot_product_attention_with_cache. cache may be NULL
 * (Option::None). query_len == 1 runs the split-K f32 decode kernel; longer
 * queries run the bf16-MFMA flash prefill (f32 in and out). out receives
 * query_len*num_heads*head_dim floats. */
int spissa_scaled_dot_product_attention_with_cache(const float *q, size_t q_len,
                                                   const float *current_k, size_t k_len,
                                                   const float *current_v, size_t v_len,
                                                   const spissa_kv_cache *cache,
                                                   const spissa_kv_attention_config *cfg,
                                                   float *out, size_t out_len);
/* Same on device buffers, asynchronous on the session stream. */
int spissa_attention_device(spissa_session *s, const float *d_q, const float *d_k,
                            const float *d_v, const spissa_kv_cache *cache,
                            const spissa_kv_attention_config *cfg, float *d_out);
/* Batched single-token decode over `batch` independent sequences in one
 * launch (the reference runs one call per sequence). d_q [batch, Hq, d],
 * d_k/d_v [batch, Hkv, d] (the new token of each sequence), caches[b] holds
 * sequence b's past; cfg->query_len must be 1. */
int spissa_attention_decode_batch_device(spissa_session *s, const float *d_q, const float *d_k,
                                         const float *d_v, const spissa_kv_cache *const *caches,
                                         size_t batch, const spissa_kv_attention_config *cfg,
                                         float *d_out);
/* One fused decode step of one layer for `batch` sequences: the RoPE of q and
 * k at position cache_len (rotary.rs:75-125 or 137-186, bit-identical to the
 * drop-in RoPE), the attention of rotary.rs:335-415 with query_len == 1, and
 * KvCache::append of the rotated key and the value (rotary.rs:226-256): the
 * call sequence of models/llama/generate.rs:373-416 and
 * models/gemma/generate.rs:247-295, in two kernel launches. d_q, d_k, d_v are
 * read-only (rotated q and k are not written back). table may be NULL (no
 * RoPE); otherwise it is a LLAMA or GEMMA table with rotary_dim == head_dim.
 * Every cache gains one token; all capacity checks run before any launch. */
int spissa_decode_step_device(spissa_session *s, const spissa_rope_table *table,
                              const float *d_q, const float *d_k, const float *d_v,
                              spissa_kv_cache *const *caches, size_t batch,
                              const spissa_kv_attention_config *cfg, float *d_out);
/* The Gemma 3 decode step of one layer in the same two launches: the
 * QK-norm of q and the new key with the [head_dim] weights d_q_norm and
 * d_k_norm (ops.rs:159-179), the Gemma RoPE from `table` (a GEMMA table over
 * the whole head), q *= q_prescale, then the attention and the append, as
 * models/gemma/generate.rs:232-295 runs them per layer (the prologue of
 * spissa_gemma_qk_prologue_device followed by spissa_decode_step_device).
 * d_q, d_k, d_v are read-only. The appended key is bit-identical to that
 * sequence's; q's sum of squares is taken as a tree (it only enters the
 * scores), so the output agrees within the attention's tolerance. */
int spissa_gemma_decode_step_device(spissa_session *s, const spissa_rope_table *table,
                                    const float *d_q, const float *d_k, const float *d_v,
                                    spissa_kv_cache *const *caches, size_t batch,
                                    const spissa_kv_attention_config *cfg, const float *d_q_norm,
                                    const float *d_k_norm, float eps, float q_prescale, float *d_out);
/* spissa_decode_step_device without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops). The split partials live in a
 * static 8 MiB device array, one copy per GPU (looked up when a session is
 * created), shared by every call of this function on that GPU: calls that
 * overlap on one GPU (on different streams) race. Splits are coarsened to
 * fit; a launch whose one-split-per-head partials (up to 16 sequences x
 * num_heads x (head_dim + 2) floats) exceed the array is rejected with
 * SPISSA_ERR_SHAPE before anything runs. Same arguments, checks and results as
 * spissa_decode_step_device. */
int spissa_decode_step_device_noalloc(spissa_session *s, const spissa_rope_table *table,
                                      const float *d_q, const float *d_k, const float *d_v,
                                      spissa_kv_cache *const *caches, size_t batch,
                                      const spissa_kv_attention_config *cfg, float *d_out);

/* Launch geometry of one attention call as the call itself computes it, on
 * the host, with no device work. No reference counterpart: it lets a caller
 * size workspaces before capturing a graph, and lets tests check the host
 * arithmetic against the kernels' index ranges without a GPU. Caches are
 * assumed under 4 GiB per buffer (the decode kernel's limit). */
typedef enum {
    SPISSA_KERNEL_DECODE = 0,       /* split-K f32 decode (query_len == 1) */
    SPISSA_KERNEL_PREFILL_BF16 = 1, /* bf16-MFMA prefill (query_len > 1) */
    SPISSA_KERNEL_GENERIC = 2       /* f32 SIMT kernel (other head dims, f32 prefill) */
} spissa_kernel_path;
typedef struct {
    int path;               /* spissa_kernel_path */
    int heads_per_block;    /* query heads sharing one K/V read (decode) or one workgroup (prefill) */
    int head_blocks;        /* head blocks per KV head */
    int keys_per_split;     /* decode: cached keys per split workgroup */
    int splits;             /* decode: splits of the longest sequence, the token's own included; prefill: key splits (1: none) */
    int token_split;        /* decode: 1 = split 0 is the new token's own split, dispatched first, and the cached
                               keys' splits are 1..splits-1; 0 = cached split 0 takes the token after its rows */
    int tiles_per_split;    /* prefill with key splits: key tiles per split */
    int tile_keys;          /* prefill: keys per tile */
    int workgroup_queries;  /* prefill: queries per workgroup */
    int block_waves;        /* prefill: waves sharing one query block's key tiles (2 = wave pairs on alternate tiles) */
    int xcd_group;          /* prefill: 1 = with key splits, the workgroups of one KV head's split share an XCD;
                               2 = unsplit windowed, each XCD takes a contiguous run of query blocks */
    long max_tiles;         /* prefill: most key tiles one unsplit workgroup visits */
    size_t workgroups;      /* attention kernel grid (decode: its first launch of <= 16 sequences) */
    size_t partial_bytes;   /* decode: split partials of the largest launch; prefill: key-split partials */
    size_t stage_bytes;     /* prefill: bf16 staging of the chunk's K and V^T */
} spissa_attention_plan;
/* past_lens[b]: cached tokens of sequence b, batch >= 1 (batch > 1 only with
 * query_len == 1); compute_units <= 0 means 256; prefill_precision as
 * spissa_session_set_prefill_precision; noalloc != 0 plans
 * spissa_decode_step_device_noalloc (SHAPE when it would reject the call). */
int spissa_plan_attention(const spissa_kv_attention_config *cfg, const size_t *past_lens, size_t batch,
                          int compute_units, int prefill_precision, int noalloc,
                          spissa_attention_plan *out);

/* One fused prefill (or chunked-prefill) step of one layer on the device,
 * the call sequence of models/llama/generate.rs:383-416 for a chunk of
 * cfg->query_len tokens: the RoPE of q and k at positions cache_len.. from
 * `table` (rotary.rs:75-125 or 137-186, bit-identical to the drop-in RoPE;
 * NULL: none), the attention of rotary.rs:335-415 over the cache's rows and
 * the chunk, and KvCache::append of the rotated keys and the values
 * (rotary.rs:226-256). In two launches: one pass appends the chunk to the
 * cache (f32 rows and the bf16 prefill operands) and stages q, then the bf16
 * MFMA attention reads every key from the cache. d_q, d_k, d_v are read-only;
 * the cache gains query_len rows. All checks run before any launch; a device
 * error (invalid softmax denominator) is reported by the next
 * spissa_session_sync(), after the rows were appended (truncate rolls them
 * back). head_dim 64, 128 or 256 with the bf16 prefill (SHAPE otherwise);
 * query_len == 1 runs the fused decode step. */
int spissa_prefill_step_device(spissa_session *s, const spissa_rope_table *table, const float *d_q,
                               const float *d_k, const float *d_v, spissa_kv_cache *cache,
                               const spissa_kv_attention_config *cfg, float *d_out);
/* The Gemma 3 prefill (or chunk) step of one layer: the QK-norm of the
 * chunk's q and k rows with the [head_dim] weights (ops.rs:159-179), the
 * Gemma RoPE from `table` (a GEMMA table over the whole head), q *= q_prescale,
 * attention and append, as models/gemma/generate.rs:232-295 runs them per
 * layer (spissa_gemma_qk_prologue_device then spissa_prefill_step_device, to
 * the bit: the norm, with the sum of squares in index order, is folded into
 * the append pass). d_q, d_k, d_v are
 * read-only. query_len == 1 runs spissa_gemma_decode_step_device. */
int spissa_gemma_prefill_step_device(spissa_session *s, const spissa_rope_table *table, const float *d_q,
                                     const float *d_k, const float *d_v, spissa_kv_cache *cache,
                                     const spissa_kv_attention_config *cfg, const float *d_q_norm,
                                     const float *d_k_norm, float eps, float q_prescale, float *d_out);

/* The attention of rotary.rs:335-415 in append-first order: the chunk's keys
 * and values are already the cache's last cfg->query_len rows (appended
 * before the call), so d_q [S, Hq, D] (rotated) attends over cache rows
 * [0, len) with query i at absolute position len - S + i. Same result as
 * spissa_attention_device(q, k, v, cache truncated to len - S, cfg) with the
 * chunk's k/v passed as current rows; this is the fused prefill step's
 * attention launch on its own. query_len > 1, bf16 prefill at head_dim 64,
 * 128 or 256 (SHAPE otherwise); len >= query_len. */
int spissa_attention_cached_device(spissa_session *s, const float *d_q, spissa_kv_cache *cache,
                                   const spissa_kv_attention_config *cfg, float *d_out);

/* ops.rs:237-291 scaled_dot_product_attention (cacheless MHA, f32). */
int spissa_scaled_dot_product_attention(const float *q, size_t q_len, const float *k,
                                        size_t k_len, const float *v, size_t v_len,
                                        size_t seq_len, size_t num_heads, size_t head_dim,
                                        int causal, float *out, size_t out_len);

/* ------------------------------------------------------------------------ */
/* Linear projections: the q/k/v/o projections either side of the path.     */
/* crates/spissa-runtime/src/streaming/linear.rs:269-576                    */
/* (streaming_tile_linear_from_model) streams the weight from the model     */
/* container chunk by chunk; here it is uploaded once and stays in HBM, and  */
/* the call computes out[batch, out] = input[batch, in] x W[out, in]^T + bias */
/* (ops.rs:62-105) in f32.                                                   */
/* ------------------------------------------------------------------------ */

/* Weight element types with a device kernel (spissa_container::DType Fp32,
 * Fp16, Bf16). */
typedef enum { SPISSA_DTYPE_F32 = 0, SPISSA_DTYPE_F16 = 1, SPISSA_DTYPE_BF16 = 2 } spissa_dtype;
typedef struct spissa_linear_weight spissa_linear_weight;
/* Uploads a row-major [out_features, in_features] weight whose little-endian
 * element bytes are `data` (what a raw chunk of the container holds).
 * data_bytes must equal out_features * in_features * element size
 * (streaming/validation.rs:258-289: InvalidTensorData otherwise). `data` may
 * be host memory or device memory of any device; work that produces it on
 * another stream must be complete before the call. */
int spissa_linear_weight_new(spissa_session *s, int dtype, size_t out_features, size_t in_features,
                             const void *data, size_t data_bytes, spissa_linear_weight **out);
/* Frees the weight after the work queued on its session. */
void spissa_linear_weight_free(spissa_linear_weight *w);
/* streaming/mod.rs:511-516 StreamingLinearConfig */
typedef struct {
    size_t batch;
    size_t in_features;
    size_t out_features;
} spissa_linear_config;
/* streaming/linear.rs:269-576 streaming_tile_linear_from_model, host buffers:
 * validate_linear_shapes (input = batch * in_features, bias = out_features:
 * Shape), then the weight shape against the config (Shape); bias may be
 * NULL (Option::None). out receives batch * out_features floats. */
int spissa_linear(const spissa_linear_weight *w, const float *input, size_t input_len,
                  const float *bias, size_t bias_len, const spissa_linear_config *cfg,
                  float *out, size_t out_len);
/* Same on device buffers (d_input [batch, in], d_bias [out] or NULL,
 * d_out [batch, out]), asynchronous on the session stream. */
int spissa_linear_device(spissa_session *s, const spissa_linear_weight *w, const float *d_input,
                         const float *d_bias, size_t batch, float *d_out);

/* ------------------------------------------------------------------------ */
/* LM head and greedy sampling: the tied embedding table as the output      */
/* projection of the last hidden row, then the argmax over the vocabulary.  */
/* ------------------------------------------------------------------------ */

/* streaming/mod.rs:186-236 lm_head_logits_parallel (f32 table) and
 * streaming/mod.rs:238-287 lm_head_logits_parallel_bf16 (bf16 table):
 * logits[v] = sum_h last_hidden[h] * table[v, h], with the table a
 * [vocab_size, hidden] spissa_linear_weight of dtype F32 or BF16 (other
 * dtypes: InvalidTensorData). last_hidden_len must equal hidden and
 * logits_len vocab_size (Shape otherwise; the reference indexes past such
 * buffers instead). Host buffers, synchronous. */
int spissa_lm_head_logits(const spissa_linear_weight *table, const float *last_hidden,
                          size_t last_hidden_len, float *logits, size_t logits_len);
/* ops.rs:309-324 sample_argmax (excluded < 0: Option::None) and
 * ops.rs:326-348 sample_argmax_excluding (excluded >= 0: Some(excluded)) over
 * host logits, on the session's device: the first maximal index, with the
 * reference's NaN and tie behaviour. n == 0: InvalidTensorData
 * ("cannot sample from empty logits"). n <= INT32_MAX - 1024 (Shape). */
int spissa_sample_argmax(spissa_session *s, const float *logits, size_t n, int64_t excluded,
                         size_t *token);
/* Same over device logits; the index is written to d_token[0] (int32). */
int spissa_argmax_device(spissa_session *s, const float *d_logits, size_t n, int64_t excluded,
                         int32_t *d_token);
/* The greedy decode tail on the device: d_logits [vocab] = table x d_hidden
 * [hidden], then, unless d_token is NULL, d_token[0] = the argmax as above. */
int spissa_lm_head_device(spissa_session *s, const spissa_linear_weight *table, const float *d_hidden,
                          int64_t excluded, float *d_logits, int32_t *d_token);

/* ------------------------------------------------------------------------ */
/* The attention sublayer of one layer on the device, in the reference's    */
/* order (models/gemma/generate.rs:178-312, models/llama/generate.rs:200-450): */
/* input RMSNorm, q/k/v projections, QK-norm (Gemma), RoPE at the cache's    */
/* next positions, q prescale, attention over cache + current rows, append   */
/* of the rotated k and v, o projection, post-attention RMSNorm (Gemma).     */
/* ------------------------------------------------------------------------ */
typedef struct {
    size_t hidden;
    size_t q_heads;
    size_t kv_heads;
    size_t head_dim;
    const spissa_linear_weight *q_weight; /* [q_heads * head_dim, hidden] */
    const spissa_linear_weight *k_weight; /* [kv_heads * head_dim, hidden] */
    const spissa_linear_weight *v_weight; /* [kv_heads * head_dim, hidden] */
    const spissa_linear_weight *o_weight; /* [hidden, q_heads * head_dim] */
    const float *d_input_norm;  /* [hidden] RMSNorm multipliers (Gemma's 1 + w), or NULL: none */
    const float *d_q_norm;      /* [head_dim] QK-norm multipliers, or NULL (then d_k_norm too) */
    const float *d_k_norm;
    const float *d_post_norm;   /* [hidden] post-attention RMSNorm multipliers, or NULL */
    float eps;                  /* RMSNorm epsilon of all the norms */
    const spissa_rope_table *rope; /* the layer's LLAMA or GEMMA table over the whole head, or NULL */
    float q_prescale;           /* models/gemma/generate.rs:275; must be 1 without the QK-norm */
    int causal;
    size_t window;              /* sliding window (0: none) */
} spissa_attention_layer;
/* d_x [seq_len, hidden] -> d_out [seq_len, hidden], asynchronous on the
 * session stream. RoPE positions start at the cache's length (0 without a
 * cache); with a cache the rotated k and v are appended, which must fit. The
 * cache must belong to the session. All checks run before any launch. */
int spissa_attention_sublayer_device(spissa_session *s, const spissa_attention_layer *layer,
                                     const float *d_x, size_t seq_len, spissa_kv_cache *cache,
                                     float *d_out);

/* Streaming-read ceiling (no reference counterpart): reads the `bytes` bytes
 * of d_buf once with 16-byte non-temporal loads, as the decode kernels read
 * the cache, asynchronously on the session stream; timing a run of these
 * gives the achievable read bandwidth the decode figures are compared with.
 * d_buf 16-byte aligned, bytes a multiple of 16 (SHAPE otherwise); d_sink is
 * one float the kernel may write. */
int spissa_hbm_read_probe_device(spissa_session *s, const void *d_buf, size_t bytes, float *d_sink);
/* Dense bf16 MFMA ceiling (no reference counterpart): two four-wave
 * workgroups per CU, each wave issuing rounds x 8 independent
 * v_mfma_f32_32x32x16_bf16 from registers, asynchronously on the session
 * stream; *flop receives the launch's FLOP count (host pointer). Timing it
 * gives the MFMA rate the device sustains, clock and power limits included,
 * which the prefill figures are compared with. rounds > 0 (SHAPE otherwise);
 * d_sink is one float the kernel may write. */
int spissa_mfma_rate_probe_device(spissa_session *s, int rounds, float *d_sink, double *flop);

/* Prefill arithmetic for query_len > 1: SPISSA_PREFILL_BF16 (default) runs
 * the MFMA kernel; SPISSA_PREFILL_F32 runs the f32 SIMT kernel. */
typedef enum { SPISSA_PREFILL_BF16 = 0, SPISSA_PREFILL_F32 = 1 } spissa_prefill_precision;
int spissa_session_set_prefill_precision(spissa_session *s, int precision);

#ifdef __cplusplus
}
#endif
#endif /* SPISSA_HIP_H */
