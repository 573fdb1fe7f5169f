/*
 * spissa_oracle.c -- CPU restatement of the Spissa runtime's attention path.
 *
 * TEST INFRASTRUCTURE ONLY (see spissa_oracle.h). The GPU product never links
 * this file; tests, smoke() and bench.py's cpu_baseline use it as the checker.
 *
 * Build: gcc -O2 -fno-fast-math -ffp-contract=off -fno-builtin-sinf
 *        -fno-builtin-cosf (see oracle/Makefile). Every f32 expression below
 * keeps the operand order of the Rust source it cites so that, with
 * contraction off, each intermediate is rounded exactly where Rust rounds it.
 */
#include "spissa_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_err[512];

const char *or_last_error(void) { return g_err; }

static int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

static int mul_ovf(size_t a, size_t b, size_t *out) {
    return __builtin_mul_overflow(a, b, out);
}

/* rotary.rs:17-38 gpt_neox_rotary_dim */
int or_gpt_neox_rotary_dim(size_t head_dim, float rotary_pct, size_t *out) {
    if (head_dim == 0) return fail(OR_SHAPE, "head_dim must be greater than zero");
    if (!isfinite(rotary_pct) || rotary_pct <= 0.0f || rotary_pct > 1.0f)
        return fail(OR_INVALID, "rotary_pct must be finite and in (0, 1], got %g", rotary_pct);
    float prod = (float)head_dim * rotary_pct;
    size_t dim = (size_t)prod; /* Rust `as usize`: truncation toward zero */
    if (dim % 2 != 0) dim -= 1;
    if (dim == 0) return fail(OR_SHAPE, "rotary_pct %g produces zero even rotary dim", rotary_pct);
    *out = dim;
    return OR_OK;
}

/* rotary.rs:454-465 rotary_angle (llama / neox angle, optional LongRoPE divisor). */
static float rotary_angle(size_t absolute_pos, size_t pair, size_t rotary_dim, float base,
                          const float *freq_scale, size_t freq_scale_len) {
    float exponent = (float)(2 * pair) / (float)rotary_dim;
    float scale = (freq_scale != NULL && pair < freq_scale_len) ? freq_scale[pair] : 1.0f;
    float inv_freq = 1.0f / (powf(base, exponent) * scale);
    return (float)absolute_pos * inv_freq;
}

void or_llama_cos_sin(size_t absolute_pos, size_t pair, size_t rotary_dim, float base,
                      float freq_scale, float *cos_out, float *sin_out) {
    float angle = rotary_angle(absolute_pos, pair, rotary_dim, base, &freq_scale, 1);
    *cos_out = cosf(angle);
    *sin_out = sinf(angle);
}

/* rotary.rs:188-193 gemma_rotary_cos_sin, with rotary.rs:168 scaled_pos. */
static void gemma_cos_sin(float scaled_pos, size_t pair, size_t rotary_dim, float base,
                          float *c, float *s) {
    float exponent = (float)(2 * pair) / (float)rotary_dim;
    float inv_freq = 1.0f / powf(base, exponent);
    float angle = scaled_pos * inv_freq;
    *c = cosf(angle);
    *s = sinf(angle);
}

void or_gemma_cos_sin(size_t absolute_pos, size_t pair, size_t rotary_dim, float base,
                      float position_divisor, float *cos_out, float *sin_out) {
    float scaled_pos = (float)absolute_pos / position_divisor;
    gemma_cos_sin(scaled_pos, pair, rotary_dim, base, cos_out, sin_out);
}

/* rotary.rs:467-481 rotate_neox_pair (rotate-half: dim `pair` against `pair + half`). */
static void rotate_pair(float *v, size_t row_start, size_t pair, size_t half, float c, float s) {
    size_t a = row_start + pair, b = row_start + pair + half;
    float first = v[a], second = v[b];
    v[a] = first * c - second * s;
    v[b] = second * c + first * s;
}

/* rotary.rs:417-452 validate_rotary_inputs */
static int validate_rotary_inputs(size_t q_len, size_t k_len, const or_rotary_config *c) {
    size_t expected;
    if (mul_ovf(c->seq_len, c->num_heads, &expected) || mul_ovf(expected, c->head_dim, &expected))
        return fail(OR_SHAPE, "rotary input length overflow");
    if (q_len != expected || k_len != expected)
        return fail(OR_SHAPE, "rotary Q/K shape mismatch: expected %zu, got q=%zu, k=%zu", expected,
                    q_len, k_len);
    if (c->seq_len == 0 || c->num_heads == 0 || c->head_dim == 0)
        return fail(OR_SHAPE, "rotary dimensions must be non-zero");
    if (c->rotary_dim == 0 || c->rotary_dim > c->head_dim || c->rotary_dim % 2 != 0)
        return fail(OR_SHAPE, "rotary_dim must be even and in 1..=head_dim, got %zu", c->rotary_dim);
    if (!isfinite(c->base) || c->base <= 0.0f)
        return fail(OR_INVALID, "rotary base must be finite and positive, got %g", c->base);
    return OR_OK;
}

/* rotary.rs:45-69 apply_gpt_neox_rotary_inplace */
int or_apply_gpt_neox_rotary_inplace(float *q, size_t q_len, float *k, size_t k_len,
                                     const or_rotary_config *cfg) {
    int st = validate_rotary_inputs(q_len, k_len, cfg);
    if (st) return st;
    size_t half = cfg->rotary_dim / 2;
    for (size_t pos = 0; pos < cfg->seq_len; ++pos) {
        size_t abs_pos;
        if (__builtin_add_overflow(cfg->position_offset, pos, &abs_pos))
            return fail(OR_SHAPE, "rotary absolute position overflow");
        for (size_t head = 0; head < cfg->num_heads; ++head) {
            size_t row = (pos * cfg->num_heads + head) * cfg->head_dim;
            for (size_t pair = 0; pair < half; ++pair) {
                float angle = rotary_angle(abs_pos, pair, cfg->rotary_dim, cfg->base, NULL, 0);
                float c = cosf(angle);
                float s = sinf(angle);
                rotate_pair(q, row, pair, half, c, s);
                rotate_pair(k, row, pair, half, c, s);
            }
        }
    }
    return OR_OK;
}

/* The Rust code indexes past the head row when 2*(rotary_dim/2) > head_dim
 * (slice panic or a write into the next head); the oracle reports Shape. */
static int guard_half(size_t half, const or_rotary_config *cfg) {
    if (cfg->seq_len > 0 && 2 * half > cfg->head_dim)
        return fail(OR_SHAPE, "rotary_dim %zu exceeds head_dim %zu", cfg->rotary_dim, cfg->head_dim);
    return OR_OK;
}

/* rotary.rs:75-125 apply_llama_rotary_inplace */
int or_apply_llama_rotary_inplace(float *q, size_t q_len, float *k, size_t k_len,
                                  size_t q_heads, size_t k_heads, const or_rotary_config *cfg,
                                  const float *freq_scale, size_t freq_scale_len) {
    if (q_heads == 0 || k_heads == 0) return fail(OR_SHAPE, "heads must be > 0");
    size_t eq = cfg->seq_len * q_heads * cfg->head_dim;
    size_t ek = cfg->seq_len * k_heads * cfg->head_dim;
    if (q_len != eq || k_len != ek)
        return fail(OR_SHAPE, "rotary shape mismatch: q=%zu, expected=%zu, k=%zu, expected=%zu", q_len,
                    eq, k_len, ek);
    size_t half = cfg->rotary_dim / 2;
    int st = guard_half(half, cfg);
    if (st) return st;
    for (size_t pos = 0; pos < cfg->seq_len; ++pos) {
        size_t abs_pos = cfg->position_offset + pos;
        for (size_t head = 0; head < q_heads; ++head) {
            size_t row = (pos * q_heads + head) * cfg->head_dim;
            for (size_t pair = 0; pair < half; ++pair) {
                float angle =
                    rotary_angle(abs_pos, pair, cfg->rotary_dim, cfg->base, freq_scale, freq_scale_len);
                float c = cosf(angle);
                float s = sinf(angle);
                rotate_pair(q, row, pair, half, c, s);
            }
        }
        for (size_t head = 0; head < k_heads; ++head) {
            size_t row = (pos * k_heads + head) * cfg->head_dim;
            for (size_t pair = 0; pair < half; ++pair) {
                float angle =
                    rotary_angle(abs_pos, pair, cfg->rotary_dim, cfg->base, freq_scale, freq_scale_len);
                float c = cosf(angle);
                float s = sinf(angle);
                rotate_pair(k, row, pair, half, c, s);
            }
        }
    }
    return OR_OK;
}

/* rotary.rs:137-186 apply_gemma_rotary_inplace */
int or_apply_gemma_rotary_inplace(float *q, size_t q_len, float *k, size_t k_len,
                                  size_t q_heads, size_t k_heads, const or_rotary_config *cfg,
                                  float position_divisor) {
    if (q_heads == 0 || k_heads == 0) return fail(OR_SHAPE, "heads must be > 0");
    if (!isfinite(position_divisor) || position_divisor <= 0.0f)
        return fail(OR_INVALID, "gemma rotary position_divisor must be finite and positive, got %g",
                    position_divisor);
    size_t eq = cfg->seq_len * q_heads * cfg->head_dim;
    size_t ek = cfg->seq_len * k_heads * cfg->head_dim;
    if (q_len != eq || k_len != ek)
        return fail(OR_SHAPE, "gemma rotary shape mismatch: q=%zu, expected=%zu, k=%zu, expected=%zu",
                    q_len, eq, k_len, ek);
    size_t half = cfg->rotary_dim / 2;
    int st = guard_half(half, cfg);
    if (st) return st;
    for (size_t pos = 0; pos < cfg->seq_len; ++pos) {
        size_t abs_pos = cfg->position_offset + pos;
        float scaled_pos = (float)abs_pos / position_divisor;
        for (size_t head = 0; head < q_heads; ++head) {
            size_t row = (pos * q_heads + head) * cfg->head_dim;
            for (size_t pair = 0; pair < half; ++pair) {
                float c, s;
                gemma_cos_sin(scaled_pos, pair, cfg->rotary_dim, cfg->base, &c, &s);
                rotate_pair(q, row, pair, half, c, s);
            }
        }
        for (size_t head = 0; head < k_heads; ++head) {
            size_t row = (pos * k_heads + head) * cfg->head_dim;
            for (size_t pair = 0; pair < half; ++pair) {
                float c, s;
                gemma_cos_sin(scaled_pos, pair, cfg->rotary_dim, cfg->base, &c, &s);
                rotate_pair(k, row, pair, half, c, s);
            }
        }
    }
    return OR_OK;
}

/* rotary.rs:206-224 KvCache::new */
or_kv_cache *or_kv_new(size_t num_heads, size_t head_dim, size_t max_seq_len, int *status) {
    if (num_heads == 0 || head_dim == 0 || max_seq_len == 0) {
        *status = fail(OR_SHAPE, "KV cache dimensions must be non-zero");
        return NULL;
    }
    size_t cap;
    if (mul_ovf(max_seq_len, num_heads, &cap) || mul_ovf(cap, head_dim, &cap) ||
        cap > ((size_t)1 << 60) / sizeof(float)) {
        *status = fail(OR_SHAPE, "KV cache capacity overflow");
        return NULL;
    }
    or_kv_cache *c = (or_kv_cache *)calloc(1, sizeof *c);
    c->num_heads = num_heads;
    c->head_dim = head_dim;
    c->max_seq_len = max_seq_len;
    c->keys = (float *)malloc(cap * sizeof(float));
    c->values = (float *)malloc(cap * sizeof(float));
    if (!c->keys || !c->values) {
        or_kv_free(c);
        *status = fail(OR_SHAPE, "KV cache allocation failed");
        return NULL;
    }
    *status = OR_OK;
    return c;
}

void or_kv_free(or_kv_cache *c) {
    if (!c) return;
    free(c->keys);
    free(c->values);
    free(c);
}

static size_t token_width(const or_kv_cache *c) { return c->num_heads * c->head_dim; }

/* rotary.rs:226-256 KvCache::append -- validates everything before mutating. */
int or_kv_append(or_kv_cache *c, const float *keys, size_t keys_len, const float *values,
                 size_t values_len, size_t token_count) {
    if (token_count == 0) return fail(OR_SHAPE, "KV cache append token_count must be greater than zero");
    size_t n;
    if (mul_ovf(token_count, token_width(c), &n)) return fail(OR_SHAPE, "KV append length overflow");
    if (keys_len != n || values_len != n)
        return fail(OR_SHAPE, "KV append shape mismatch: expected %zu, got keys=%zu, values=%zu", n,
                    keys_len, values_len);
    size_t new_len;
    if (__builtin_add_overflow(c->len, token_count, &new_len))
        return fail(OR_SHAPE, "KV cache length overflow");
    if (new_len > c->max_seq_len)
        return fail(OR_SHAPE, "KV cache capacity exceeded: append would set len %zu, max_seq_len %zu",
                    new_len, c->max_seq_len);
    size_t off = c->len * token_width(c);
    memcpy(c->keys + off, keys, n * sizeof(float));
    memcpy(c->values + off, values, n * sizeof(float));
    c->len = new_len;
    return OR_OK;
}

/* rotary.rs:258-262 */
void or_kv_clear(or_kv_cache *c) { c->len = 0; }

/* rotary.rs:264-278 */
int or_kv_truncate(or_kv_cache *c, size_t len) {
    if (len > c->len) return fail(OR_SHAPE, "KV cache truncate cannot grow from %zu to %zu", c->len, len);
    c->len = len;
    return OR_OK;
}

/* rotary.rs:280-285 (saturating) */
size_t or_kv_resident_bytes(const or_kv_cache *c) {
    size_t r;
    if (mul_ovf(c->len, token_width(c), &r) || mul_ovf(r, 2, &r) || mul_ovf(r, sizeof(float), &r))
        return (size_t)-1;
    return r;
}

size_t or_kv_len(const or_kv_cache *c) { return c->len; }
const float *or_kv_keys(const or_kv_cache *c) { return c->keys; }
const float *or_kv_values(const or_kv_cache *c) { return c->values; }

/* rotary.rs:549-569 softmax_inplace */
static int softmax_inplace(float *x, size_t n) {
    if (n == 0) return OR_OK;
    float max = -INFINITY;
    for (size_t i = 0; i < n; ++i) max = fmaxf(max, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float e = expf(x[i] - max);
        x[i] = e;
        sum += e;
    }
    if (sum == 0.0f || !isfinite(sum)) return fail(OR_INVALID, "softmax produced invalid denominator");
    for (size_t i = 0; i < n; ++i) x[i] /= sum;
    return OR_OK;
}

/* rotary.rs:577-599 kv_row */
static const float *kv_row(const or_kv_cache *cache, const float *cache_buf, const float *current,
                           size_t past_len, size_t key_pos, size_t kv_head, size_t kv_heads,
                           size_t head_dim) {
    (void)cache;
    if (key_pos < past_len) return cache_buf + (key_pos * kv_heads + kv_head) * head_dim;
    size_t cur = key_pos - past_len;
    return current + (cur * kv_heads + kv_head) * head_dim;
}

/* rotary.rs:483-547 validate_kv_attention_inputs */
static int validate_kv(size_t q_len, size_t k_len, size_t v_len, const or_kv_cache *cache,
                       const or_kv_attention_config *c) {
    if (c->query_len == 0 || c->num_heads == 0 || c->kv_heads == 0 || c->head_dim == 0)
        return fail(OR_SHAPE, "KV attention dimensions must be non-zero");
    if (c->num_heads % c->kv_heads != 0)
        return fail(OR_SHAPE, "query heads %zu must be a multiple of key/value heads %zu", c->num_heads,
                    c->kv_heads);
    size_t eq, ekv;
    if (mul_ovf(c->query_len, c->num_heads, &eq) || mul_ovf(eq, c->head_dim, &eq))
        return fail(OR_SHAPE, "KV attention current length overflow");
    if (mul_ovf(c->query_len, c->kv_heads, &ekv) || mul_ovf(ekv, c->head_dim, &ekv))
        return fail(OR_SHAPE, "KV attention current length overflow");
    if (q_len != eq || k_len != ekv || v_len != ekv)
        return fail(OR_SHAPE, "KV attention shape mismatch: expected q=%zu, k/v=%zu, got q=%zu, k=%zu, v=%zu",
                    eq, ekv, q_len, k_len, v_len);
    if (cache && (cache->num_heads != c->kv_heads || cache->head_dim != c->head_dim))
        return fail(OR_SHAPE, "KV cache shape mismatch");
    return OR_OK;
}

/* rotary.rs:335-415 scaled_dot_product_attention_with_cache.
 * Extension (not in the reference): window > 0 additionally masks keys with
 * key_pos + window <= query_abs_pos (HF sliding-window rule i-W < j <= i).
 * window = 0 is exactly the reference. */
int or_sdpa_with_cache(const float *q, size_t q_len, const float *cur_k, size_t k_len,
                       const float *cur_v, size_t v_len, const or_kv_cache *cache,
                       const or_kv_attention_config *cfg, float *out, size_t out_len) {
    int st = validate_kv(q_len, k_len, v_len, cache, cfg);
    if (st) return st;
    if (out_len != q_len) return fail(OR_SHAPE, "output length %zu != %zu", out_len, q_len);
    size_t past_len = cache ? cache->len : 0;
    size_t key_len;
    if (__builtin_add_overflow(past_len, cfg->query_len, &key_len))
        return fail(OR_SHAPE, "KV attention key length overflow");
    size_t d = cfg->head_dim;
    float scale = 1.0f / sqrtf((float)d);
    float *scores = (float *)malloc((key_len ? key_len : 1) * sizeof(float));
    float *res = (float *)calloc(q_len ? q_len : 1, sizeof(float));
    size_t repeats = cfg->num_heads / cfg->kv_heads;
    const float *ck = cache ? cache->keys : NULL, *cv = cache ? cache->values : NULL;

    for (size_t qp = 0; qp < cfg->query_len; ++qp) {
        size_t q_abs = past_len + qp;
        for (size_t head = 0; head < cfg->num_heads; ++head) {
            const float *qrow = q + (qp * cfg->num_heads + head) * d;
            size_t kv_head = head / repeats;
            for (size_t kp = 0; kp < key_len; ++kp) {
                if (cfg->causal && kp > q_abs) {
                    scores[kp] = -INFINITY;
                    continue;
                }
                if (cfg->window > 0 && kp + cfg->window <= q_abs) {
                    scores[kp] = -INFINITY;
                    continue;
                }
                const float *krow = kv_row(cache, ck, cur_k, past_len, kp, kv_head, cfg->kv_heads, d);
                float dot = 0.0f;
                for (size_t i = 0; i < d; ++i) dot += qrow[i] * krow[i];
                scores[kp] = dot * scale;
            }
            st = softmax_inplace(scores, key_len);
            if (st) {
                free(scores);
                free(res);
                return st;
            }
            float *orow = res + (qp * cfg->num_heads + head) * d;
            for (size_t i = 0; i < d; ++i) orow[i] = 0.0f;
            for (size_t kp = 0; kp < key_len; ++kp) {
                float p = scores[kp];
                const float *vrow = kv_row(cache, cv, cur_v, past_len, kp, kv_head, cfg->kv_heads, d);
                for (size_t i = 0; i < d; ++i) orow[i] += p * vrow[i];
            }
        }
    }
    memcpy(out, res, q_len * sizeof(float));
    free(scores);
    free(res);
    return OR_OK;
}

/* ops.rs:159-179 rms_norm */
int or_rms_norm(const float *x, size_t x_len, const float *w, size_t w_len, size_t rows,
                size_t cols, float eps, float *out) {
    if (x_len != rows * cols || w_len != cols)
        return fail(OR_SHAPE, "rms_norm shape mismatch: x=%zu, rows=%zu, cols=%zu, weight=%zu", x_len,
                    rows, cols, w_len);
    for (size_t r = 0; r < rows; ++r) {
        const float *row = x + r * cols;
        float acc = 0.0f;
        for (size_t c = 0; c < cols; ++c) acc += row[c] * row[c];
        float mean_square = acc / (float)cols;
        float inv_rms = 1.0f / sqrtf(mean_square + eps);
        for (size_t c = 0; c < cols; ++c) out[r * cols + c] = row[c] * inv_rms * w[c];
    }
    return OR_OK;
}

/* ops.rs:202-232 softmax_rows */
int or_softmax_rows(const float *logits, size_t len, size_t rows, size_t cols, float *out) {
    if (len != rows * cols)
        return fail(OR_SHAPE, "softmax len %zu does not match rows*cols = %zu", len, rows * cols);
    for (size_t r = 0; r < rows; ++r) {
        const float *row = logits + r * cols;
        float max = -INFINITY;
        for (size_t c = 0; c < cols; ++c) max = fmaxf(max, row[c]);
        float sum = 0.0f;
        for (size_t c = 0; c < cols; ++c) {
            float e = expf(row[c] - max);
            out[r * cols + c] = e;
            sum += e;
        }
        if (sum == 0.0f || !isfinite(sum)) return fail(OR_INVALID, "softmax produced invalid denominator");
        for (size_t c = 0; c < cols; ++c) out[r * cols + c] /= sum;
    }
    return OR_OK;
}

/* ops.rs:237-291 scaled_dot_product_attention (cacheless MHA; the tests' full-recompute oracle) */
int or_scaled_dot_product_attention(const float *q, const float *k, const float *v, size_t len,
                                    size_t seq_len, size_t num_heads, size_t head_dim,
                                    int causal, float *out) {
    size_t expected = seq_len * num_heads * head_dim;
    if (len != expected) return fail(OR_SHAPE, "attention shape mismatch: expected %zu", expected);
    float scale = 1.0f / sqrtf((float)head_dim);
    float *scores = (float *)malloc((seq_len ? seq_len : 1) * sizeof(float));
    float *probs = (float *)malloc((seq_len ? seq_len : 1) * sizeof(float));
    for (size_t pos = 0; pos < seq_len; ++pos) {
        for (size_t head = 0; head < num_heads; ++head) {
            for (size_t kp = 0; kp < seq_len; ++kp) {
                if (causal && kp > pos) {
                    scores[kp] = -INFINITY;
                    continue;
                }
                float dot = 0.0f;
                for (size_t i = 0; i < head_dim; ++i) {
                    size_t qi = (pos * num_heads + head) * head_dim + i;
                    size_t ki = (kp * num_heads + head) * head_dim + i;
                    dot += q[qi] * k[ki];
                }
                scores[kp] = dot * scale;
            }
            int st = or_softmax_rows(scores, seq_len, 1, seq_len, probs);
            if (st) {
                free(scores);
                free(probs);
                return st;
            }
            for (size_t i = 0; i < head_dim; ++i) {
                size_t oi = (pos * num_heads + head) * head_dim + i;
                float value = 0.0f;
                for (size_t kp = 0; kp < seq_len; ++kp)
                    value += probs[kp] * v[(kp * num_heads + head) * head_dim + i];
                out[oi] = value;
            }
        }
    }
    free(scores);
    free(probs);
    return OR_OK;
}

/* models/gemma/model.rs:46-51 is_global_layer */
int or_is_global_layer(size_t layer_idx, size_t pattern) {
    if (pattern <= 1) return 1;
    return (layer_idx + 1) % pattern == 0;
}

/* models/gemma/generate.rs:230-278: QK-norm (rms_norm per head row), dual RoPE
 * through apply_gemma_rotary_inplace, then the Q prescale
 * attn_scale * sqrt(head_dim) with attn_scale = 1/sqrt(query_pre_attn_scalar)
 * (models/gemma/api.rs:115,136). The caller picks (base, divisor) by layer kind. */
int or_gemma_qk_prologue(float *q, size_t q_len, float *k, size_t k_len, size_t seq_len,
                         size_t q_heads, size_t kv_heads, size_t head_dim, const float *q_norm,
                         const float *k_norm, float eps, float rope_base,
                         float position_divisor, size_t position_offset,
                         float query_pre_attn_scalar) {
    float *qn = (float *)malloc((q_len ? q_len : 1) * sizeof(float));
    float *kn = (float *)malloc((k_len ? k_len : 1) * sizeof(float));
    int st = or_rms_norm(q, q_len, q_norm, head_dim, seq_len * q_heads, head_dim, eps, qn);
    if (!st) st = or_rms_norm(k, k_len, k_norm, head_dim, seq_len * kv_heads, head_dim, eps, kn);
    if (!st) {
        or_rotary_config rc = {seq_len, q_heads, head_dim, head_dim, rope_base, position_offset};
        st = or_apply_gemma_rotary_inplace(qn, q_len, kn, k_len, q_heads, kv_heads, &rc,
                                           position_divisor);
    }
    if (!st) {
        float attn_scale = 1.0f / sqrtf(query_pre_attn_scalar);
        float q_prescale = attn_scale * sqrtf((float)head_dim);
        for (size_t i = 0; i < q_len; ++i) qn[i] *= q_prescale;
        memcpy(q, qn, q_len * sizeof(float));
        memcpy(k, kn, k_len * sizeof(float));
    }
    free(qn);
    free(kn);
    return st;
}

typedef struct {
    size_t begin, end;
    const float *const *q, *const *k, *const *v;
    const or_kv_cache *const *caches;
    const or_kv_attention_config *cfg;
    float *const *out;
    int status;
} sdpa_job;

static void *sdpa_worker(void *arg) {
    sdpa_job *j = (sdpa_job *)arg;
    size_t ql = j->cfg->query_len * j->cfg->num_heads * j->cfg->head_dim;
    size_t kl = j->cfg->query_len * j->cfg->kv_heads * j->cfg->head_dim;
    for (size_t u = j->begin; u < j->end && j->status == OR_OK; ++u)
        j->status = or_sdpa_with_cache(j->q[u], ql, j->k[u], kl, j->v[u], kl, j->caches[u], j->cfg,
                                       j->out[u], ql);
    return NULL;
}

int or_sdpa_many_threads(size_t units, const float *const *q, const float *const *k,
                         const float *const *v, const or_kv_cache *const *caches,
                         const or_kv_attention_config *cfg, float *const *out, int threads) {
    if (threads < 1) threads = 1;
    if ((size_t)threads > units) threads = (int)(units ? units : 1);
    pthread_t tid[256];
    sdpa_job jobs[256];
    if (threads > 256) threads = 256;
    size_t per = (units + threads - 1) / threads;
    for (int t = 0; t < threads; ++t) {
        size_t b = t * per, e = b + per > units ? units : b + per;
        jobs[t] = (sdpa_job){b, e, q, k, v, caches, cfg, out, OR_OK};
        pthread_create(&tid[t], NULL, sdpa_worker, &jobs[t]);
    }
    int st = OR_OK;
    for (int t = 0; t < threads; ++t) {
        pthread_join(tid[t], NULL);
        if (jobs[t].status != OR_OK && st == OR_OK) st = jobs[t].status;
    }
    return st;
}

/* ---------------------------------------------------------------- linear */

float or_bf16_to_f32(uint16_t bits) {
    const uint32_t u = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

float or_fp16_to_f32(uint16_t bits) {
    const uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    const unsigned exp = (bits >> 10) & 0x1fu, frac = bits & 0x3ffu;
    uint32_t u;
    if (exp == 0x1f) {
        u = sign | 0x7f800000u | ((uint32_t)frac << 13); /* inf, nan */
    } else if (exp != 0) {
        u = sign | ((exp + 112u) << 23) | ((uint32_t)frac << 13); /* normal: rebias 15 -> 127 */
    } else {
        /* zero or subnormal: frac * 2^-24, exact in f32 */
        float v = ldexpf((float)frac, -24);
        memcpy(&u, &v, sizeof u);
        u |= sign;
    }
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

uint16_t or_f32_to_bf16_rne(float x) {
    uint32_t b;
    memcpy(&b, &x, sizeof b);
    if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x0040u); /* NaN stays NaN */
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

static float weight_at(const void *w, int dtype, size_t i) {
    switch (dtype) {
        case OR_DTYPE_BF16: return or_bf16_to_f32(((const uint16_t *)w)[i]);
        case OR_DTYPE_F16: return or_fp16_to_f32(((const uint16_t *)w)[i]);
        default: return ((const float *)w)[i];
    }
}

int or_linear(const float *input, size_t input_len, const void *weight, int dtype, size_t weight_elems,
              const float *bias, size_t bias_len, size_t batch, size_t in_features,
              size_t out_features, float *out) {
    if (input_len != batch * in_features)
        return fail(OR_SHAPE, "input len %zu does not match batch*in_features = %zu", input_len,
                    batch * in_features);
    if (weight_elems != out_features * in_features)
        return fail(OR_SHAPE, "weight len %zu does not match out_features*in_features = %zu", weight_elems,
                    out_features * in_features);
    if (bias && bias_len != out_features)
        return fail(OR_SHAPE, "bias len %zu does not match out_features %zu", bias_len, out_features);
    if (dtype != OR_DTYPE_F32 && dtype != OR_DTYPE_F16 && dtype != OR_DTYPE_BF16)
        return fail(OR_INVALID, "unsupported weight dtype %d", dtype);
    for (size_t b = 0; b < batch; ++b) {
        const float *x = input + b * in_features;
        for (size_t o = 0; o < out_features; ++o) {
            float sum = bias ? bias[o] : 0.0f;
            const size_t row = o * in_features;
            for (size_t i = 0; i < in_features; ++i) sum += x[i] * weight_at(weight, dtype, row + i);
            out[b * out_features + o] = sum;
        }
    }
    return OR_OK;
}

int or_lm_head_logits(const float *last_hidden, size_t hidden_len, const void *table, int dtype,
                      size_t vocab_size, size_t hidden, float *logits) {
    if (dtype != OR_DTYPE_F32 && dtype != OR_DTYPE_BF16)
        return fail(OR_INVALID, "LM head table must be f32 or bf16 (dtype %d)", dtype);
    if (hidden_len != hidden) return fail(OR_SHAPE, "last_hidden holds %zu floats, hidden is %zu", hidden_len, hidden);
    for (size_t v = 0; v < vocab_size; ++v) {
        float sum = 0.0f;
        const size_t row = v * hidden;
        for (size_t h = 0; h < hidden; ++h) sum += last_hidden[h] * weight_at(table, dtype, row + h);
        logits[v] = sum;
    }
    return OR_OK;
}

int or_sample_argmax(const float *logits, size_t n, size_t *out) {
    if (n == 0) return fail(OR_INVALID, "cannot sample from empty logits");
    size_t best_index = 0;
    float best_value = logits[0];
    for (size_t i = 1; i < n; ++i) {
        if (logits[i] > best_value) {
            best_index = i;
            best_value = logits[i];
        }
    }
    *out = best_index;
    return OR_OK;
}

int or_sample_argmax_excluding(const float *logits, size_t n, int has_excluded, size_t excluded,
                               size_t *out) {
    if (!has_excluded || excluded >= n || n <= 1) return or_sample_argmax(logits, n, out);
    int have = 0;
    size_t best_index = 0;
    float best_value = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        if (i == excluded) continue;
        /* ops.rs:339-342: keep the best only while value <= best */
        if (have && logits[i] <= best_value) continue;
        have = 1;
        best_index = i;
        best_value = logits[i];
    }
    if (!have) return fail(OR_INVALID, "cannot sample from empty logits");
    *out = best_index;
    return OR_OK;
}

