// abi.hip -- the extern "C" boundary (include/spissa_hip.h): sessions, the
// device-resident KV cache, validation with the reference's error contract,
// host-side RoPE tables, and dispatch to the gfx950 kernels.
//
// Validation order and messages follow crates/spissa-runtime/src/rotary.rs
// and ops.rs so that a caller sees the same RuntimeError variant for the same
// bad input; every check runs before anything is mutated.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

#include "internal.hpp"

using namespace spissa;

// ------------------------------------------------------------------------
// errors
// ------------------------------------------------------------------------
static thread_local char g_err[1024];

static int set_err(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

#define HIP_TRY(expr)                                                                       \
  do {                                                                                      \
    hipError_t e_ = (expr);                                                                 \
    if (e_ != hipSuccess)                                                                   \
      return set_err(SPISSA_ERR_DEVICE, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                     __FILE__, __LINE__);                                                   \
  } while (0)

#define ST_TRY(expr)        \
  do {                      \
    int st_ = (expr);       \
    if (st_) return st_;    \
  } while (0)

#define GUARD_BEGIN try {
#define GUARD_END                                                                 \
  }                                                                               \
  catch (const std::bad_alloc &) {                                                \
    return set_err(SPISSA_ERR_DEVICE, "host allocation failed");                  \
  }                                                                               \
  catch (...) {                                                                   \
    return set_err(SPISSA_ERR_DEVICE, "unexpected C++ exception at the C boundary"); \
  }

static bool mul_ovf(size_t a, size_t b, size_t *out) { return __builtin_mul_overflow(a, b, out); }

extern "C" const char *spissa_last_error(void) { return g_err; }
extern "C" const char *spissa_version(void) { return "spissa-hip 0.1.0 (gfx950)"; }

// ------------------------------------------------------------------------
// sessions and workspace
// ------------------------------------------------------------------------
struct DevBuf {
  void *p = nullptr;
  size_t bytes = 0;
};

// Decode partials of spissa_decode_step_device_noalloc: a static device
// array, one copy per GPU, held until the process ends and shared by every
// such call on that GPU (calls that overlap on one GPU race). Nothing in it
// needs clearing: a split writes its whole entry before the merge reads it,
// and the merge reads only the splits that ran. Host code takes its device
// address from hipGetSymbolAddress (scratch_address) and never passes the
// array's name to a kernel.
constexpr size_t kScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

static std::mutex g_scratch_mu;
static std::vector<float *> g_scratch_addr;  // per device

// The device address of `scratch` on `device`, which must be current; looked
// up once per device.
static int scratch_address(int device, float **out) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if ((int)g_scratch_addr.size() <= device) g_scratch_addr.resize(device + 1, nullptr);
  if (!g_scratch_addr[device]) {
    void *p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return set_err(SPISSA_ERR_DEVICE, "hipGetSymbolAddress gave no address for the scratch array");
    g_scratch_addr[device] = (float *)p;
  }
  *out = g_scratch_addr[device];
  return SPISSA_OK;
}

struct spissa_session {
  int device = 0;
  hipStream_t stream = nullptr;
  bool own_stream = false;
  int *d_err = nullptr;
  DevBuf io;        // drop-in host<->device staging
  DevBuf partial;   // decode split partials
  DevBuf stage;     // prefill bf16 staging of K / V^T
  DevBuf table;     // drop-in RoPE rows
  DevBuf ppart;     // prefill key-split partials (O, then (m, l))
  DevBuf sub;       // attention sublayer intermediates (normed x, q, k, v, attention, projection)
  DevBuf amax;      // argmax partials
  DevBuf qstage;    // fused prefill step: bf16 Q operand
  float *scratch = nullptr;  // this device's copy of `scratch` (kScratchBytes)
  int cus = 256;    // compute units of the device
  // Buffers replaced by larger ones. They stay allocated until the session
  // is destroyed, so a HIP graph captured before a workspace grew still
  // replays on valid memory.
  std::vector<void *> retired;
  int prefill_precision = SPISSA_PREFILL_BF16;
  // The owner's reference plus one per cache and weight created on the
  // session: those are freed through it, so it outlives them whatever order
  // the caller releases things in.
  std::atomic<int> refs{1};
};

struct spissa_kv_cache {
  spissa_session *session = nullptr;
  size_t num_heads = 0, head_dim = 0, max_seq_len = 0, len = 0;
  float *keys = nullptr;    // [max_seq_len, H, D]
  float *values = nullptr;  // [max_seq_len, H, D]
  bf16 *kb = nullptr;       // bf16 shadow [H, cap, D], allocated at first prefill use
  bf16 *vt = nullptr;       // bf16 shadow [H, D, cap]
  size_t shadow_cap = 0;
  size_t width() const { return num_heads * head_dim; }
};

struct spissa_rope_table {
  int device = 0;
  int kind = 0;
  size_t rotary_dim = 0, half = 0, max_positions = 0;
  float *cos = nullptr, *sin = nullptr;  // [max_positions, half]
};

// Device memory cannot be allocated while `stream` is being captured into a
// HIP graph; a call that would allocate then fails with this message instead
// of a generic device error.
static int no_capture(hipStream_t stream, const char *what, size_t bytes) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(stream, &cs));
  if (cs != hipStreamCaptureStatusNone)
    return set_err(SPISSA_ERR_ARGUMENT,
                   "%s would allocate %zu bytes while the session stream is being captured into a graph; run the "
                   "same call once before capturing",
                   what, bytes);
  return SPISSA_OK;
}

static int ensure_buf(spissa_session *s, DevBuf &b, size_t bytes) {
  if (bytes <= b.bytes) return SPISSA_OK;
  ST_TRY(no_capture(s->stream, "the session workspace", bytes));
  size_t want = std::max(bytes, b.bytes + b.bytes / 2);
  want = (want + 4095) & ~(size_t)4095;
  HIP_TRY(hipSetDevice(s->device));
  void *p = nullptr;
  HIP_TRY(hipMalloc(&p, want));
  if (b.p) s->retired.push_back(b.p);
  b.p = p;
  b.bytes = want;
  return SPISSA_OK;
}

static void free_buf(DevBuf &b) {
  if (b.p) (void)hipFree(b.p);
  b.p = nullptr;
  b.bytes = 0;
}

extern "C" int spissa_session_create(int device, void *stream, spissa_session **out) {
  GUARD_BEGIN
  if (!out) return set_err(SPISSA_ERR_ARGUMENT, "out is null");
  *out = nullptr;
  int n = 0;
  HIP_TRY(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return set_err(SPISSA_ERR_DEVICE, "device %d not present (%d)", device, n);
  HIP_TRY(hipSetDevice(device));
  std::unique_ptr<spissa_session> s(new spissa_session());
  s->device = device;
  HIP_TRY(hipDeviceGetAttribute(&s->cus, hipDeviceAttributeMultiprocessorCount, device));
  ST_TRY(scratch_address(device, &s->scratch));
  if (stream) {
    s->stream = (hipStream_t)stream;
  } else {
    HIP_TRY(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
    s->own_stream = true;
  }
  HIP_TRY(hipMalloc(&s->d_err, sizeof(int)));
  HIP_TRY(hipMemsetAsync(s->d_err, 0, sizeof(int), s->stream));
  HIP_TRY(hipStreamSynchronize(s->stream));
  *out = s.release();
  return SPISSA_OK;
  GUARD_END
}

static void session_free(spissa_session *s) {
  (void)hipSetDevice(s->device);
  (void)hipStreamSynchronize(s->stream);
  free_buf(s->io);
  free_buf(s->partial);
  free_buf(s->stage);
  free_buf(s->table);
  free_buf(s->ppart);
  free_buf(s->sub);
  free_buf(s->amax);
  free_buf(s->qstage);
  for (void *p : s->retired) (void)hipFree(p);
  if (s->d_err) (void)hipFree(s->d_err);
  if (s->own_stream) (void)hipStreamDestroy(s->stream);
  delete s;
}

static void session_retain(spissa_session *s) { s->refs.fetch_add(1, std::memory_order_relaxed); }
static void session_release(spissa_session *s) {
  if (s->refs.fetch_sub(1, std::memory_order_acq_rel) == 1) session_free(s);
}

extern "C" void spissa_session_destroy(spissa_session *s) {
  if (!s) return;
  session_release(s);  // freed now, or when its last cache or weight is
}

namespace {
struct DefaultSessions {
  std::vector<spissa_session *> by_device;
  ~DefaultSessions() {
    for (auto *s : by_device) spissa_session_destroy(s);
  }
};
thread_local DefaultSessions t_default;
}  // namespace

extern "C" int spissa_default_session(spissa_session **out) {
  GUARD_BEGIN
  if (!out) return set_err(SPISSA_ERR_ARGUMENT, "out is null");
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  if ((int)t_default.by_device.size() <= dev) t_default.by_device.resize(dev + 1, nullptr);
  if (!t_default.by_device[dev]) {
    int st = spissa_session_create(dev, nullptr, &t_default.by_device[dev]);
    if (st) return st;
  }
  *out = t_default.by_device[dev];
  return SPISSA_OK;
  GUARD_END
}

extern "C" int spissa_session_sync(spissa_session *s) {
  GUARD_BEGIN
  if (!s) return set_err(SPISSA_ERR_ARGUMENT, "session is null");
  HIP_TRY(hipSetDevice(s->device));
  HIP_TRY(hipStreamSynchronize(s->stream));
  int flag = 0;
  HIP_TRY(hipMemcpy(&flag, s->d_err, sizeof(int), hipMemcpyDeviceToHost));
  if (flag) {
    HIP_TRY(hipMemsetAsync(s->d_err, 0, sizeof(int), s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    if (flag & kDevErrSoftmaxDenominator)
      return set_err(SPISSA_ERR_INVALID_TENSOR_DATA, "softmax produced invalid denominator");
    return set_err(SPISSA_ERR_DEVICE, "device error flag 0x%x", flag);
  }
  return SPISSA_OK;
  GUARD_END
}

extern "C" void *spissa_session_stream(spissa_session *s) { return s ? (void *)s->stream : nullptr; }
extern "C" int spissa_session_device(const spissa_session *s) { return s ? s->device : -1; }

extern "C" int spissa_hbm_read_probe_device(spissa_session *s, const void *d_buf, size_t bytes, float *d_sink) {
  GUARD_BEGIN
  if (!s || !d_buf || !d_sink) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  if (bytes % 16 != 0 || reinterpret_cast<uintptr_t>(d_buf) % 16 != 0)
    return set_err(SPISSA_ERR_SHAPE, "the read probe needs a 16-byte aligned buffer of a multiple of 16 bytes");
  HIP_TRY(hipSetDevice(s->device));
  HIP_TRY(launch_hbm_read(s->stream, d_buf, bytes, d_sink));
  return SPISSA_OK;
  GUARD_END
}

extern "C" int spissa_mfma_rate_probe_device(spissa_session *s, int rounds, float *d_sink, double *flop) {
  GUARD_BEGIN
  if (!s || !d_sink || !flop) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  if (rounds <= 0) return set_err(SPISSA_ERR_SHAPE, "the MFMA probe needs rounds > 0, got %d", rounds);
  HIP_TRY(hipSetDevice(s->device));
  HIP_TRY(launch_mfma_rate(s->stream, s->cus, rounds, d_sink, flop));
  return SPISSA_OK;
  GUARD_END
}

extern "C" int spissa_session_set_prefill_precision(spissa_session *s, int precision) {
  if (!s) return set_err(SPISSA_ERR_ARGUMENT, "session is null");
  if (precision != SPISSA_PREFILL_BF16 && precision != SPISSA_PREFILL_F32)
    return set_err(SPISSA_ERR_ARGUMENT, "unknown prefill precision %d", precision);
  s->prefill_precision = precision;
  return SPISSA_OK;
}

// Host-buffer staging for drop-in calls: carve `n` float regions out of s->io.
static int io_regions(spissa_session *s, std::initializer_list<size_t> sizes, float **out) {
  size_t total = 0;
  for (size_t n : sizes) total += (n + 63) & ~(size_t)63;
  int st = ensure_buf(s, s->io, std::max<size_t>(total, 64) * sizeof(float));
  if (st) return st;
  float *p = (float *)s->io.p;
  int i = 0;
  for (size_t n : sizes) {
    out[i++] = p;
    p += (n + 63) & ~(size_t)63;
  }
  return SPISSA_OK;
}

static int h2d(spissa_session *s, void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return SPISSA_OK;
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s->stream));
  return SPISSA_OK;
}
static int d2h(spissa_session *s, void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return SPISSA_OK;
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s->stream));
  return SPISSA_OK;
}
static int sync_stream(spissa_session *s) {
  HIP_TRY(hipStreamSynchronize(s->stream));
  return SPISSA_OK;
}

// ------------------------------------------------------------------------
// KV cache (rotary.rs:195-318)
// ------------------------------------------------------------------------
static int kv_validate_new(size_t num_heads, size_t head_dim, size_t max_seq_len) {
  // rotary.rs:207-215
  if (num_heads == 0 || head_dim == 0 || max_seq_len == 0)
    return set_err(SPISSA_ERR_SHAPE,
                   "KV cache dimensions must be non-zero, got num_heads=%zu, head_dim=%zu, "
                   "max_seq_len=%zu",
                   num_heads, head_dim, max_seq_len);
  size_t cap;
  if (mul_ovf(max_seq_len, num_heads, &cap) || mul_ovf(cap, head_dim, &cap) ||
      cap > ((size_t)1 << 61) / sizeof(float))
    return set_err(SPISSA_ERR_SHAPE, "KV cache capacity overflow");
  return SPISSA_OK;
}

static int kv_new_impl(spissa_session *s, size_t num_heads, size_t head_dim, size_t max_seq_len,
                       spissa_kv_cache **out) {
  if (!out) return set_err(SPISSA_ERR_ARGUMENT, "out is null");
  *out = nullptr;
  // rotary.rs:207-211
  if (num_heads == 0 || head_dim == 0 || max_seq_len == 0)
    return set_err(SPISSA_ERR_SHAPE,
                   "KV cache dimensions must be non-zero, got num_heads=%zu, head_dim=%zu, "
                   "max_seq_len=%zu",
                   num_heads, head_dim, max_seq_len);
  // rotary.rs:212-215
  size_t cap;
  if (mul_ovf(max_seq_len, num_heads, &cap) || mul_ovf(cap, head_dim, &cap) ||
      cap > ((size_t)1 << 61) / sizeof(float))
    return set_err(SPISSA_ERR_SHAPE, "KV cache capacity overflow");
  std::unique_ptr<spissa_kv_cache> c(new spissa_kv_cache());
  c->session = s;
  c->num_heads = num_heads;
  c->head_dim = head_dim;
  c->max_seq_len = max_seq_len;
  HIP_TRY(hipSetDevice(s->device));
  HIP_TRY(hipMalloc(&c->keys, cap * sizeof(float)));
  hipError_t e = hipMalloc(&c->values, cap * sizeof(float));
  if (e != hipSuccess) {
    (void)hipFree(c->keys);
    return set_err(SPISSA_ERR_DEVICE, "hipMalloc of %zu bytes failed: %s", cap * sizeof(float),
                   hipGetErrorString(e));
  }
  *out = c.release();
  session_retain(s);
  return SPISSA_OK;
}

extern "C" int spissa_kv_cache_new_in(spissa_session *s, size_t num_heads, size_t head_dim,
                                      size_t max_seq_len, spissa_kv_cache **out) {
  GUARD_BEGIN
  if (!s) return set_err(SPISSA_ERR_ARGUMENT, "session is null");
  return kv_new_impl(s, num_heads, head_dim, max_seq_len, out);
  GUARD_END
}

extern "C" int spissa_kv_cache_new(size_t num_heads, size_t head_dim, size_t max_seq_len,
                                   spissa_kv_cache **out) {
  GUARD_BEGIN
  if (!out) return set_err(SPISSA_ERR_ARGUMENT, "out is null");
  *out = nullptr;
  ST_TRY(kv_validate_new(num_heads, head_dim, max_seq_len));
  spissa_session *s = nullptr;
  ST_TRY(spissa_default_session(&s));
  return kv_new_impl(s, num_heads, head_dim, max_seq_len, out);
  GUARD_END
}

static void kv_release(spissa_kv_cache *c) {
  (void)hipSetDevice(c->session->device);
  (void)hipStreamSynchronize(c->session->stream);
  if (c->keys) (void)hipFree(c->keys);
  if (c->values) (void)hipFree(c->values);
  if (c->kb) (void)hipFree(c->kb);
  if (c->vt) (void)hipFree(c->vt);
}

extern "C" void spissa_kv_cache_free(spissa_kv_cache *c) {
  if (!c) return;
  kv_release(c);
  spissa_session *s = c->session;
  delete c;
  session_release(s);
}

// Converts rows [first, first + n) of the cache into the bf16 shadow, on `st`.
static int shadow_update(spissa_kv_cache *c, size_t first, size_t n, hipStream_t st) {
  if (!c->kb || n == 0) return SPISSA_OK;
  const size_t w = c->width();
  HIP_TRY(launch_stage_bf16(st, c->keys + first * w, c->values + first * w, n, n, c->num_heads, c->head_dim,
                            c->kb, c->vt, first, c->shadow_cap));
  return SPISSA_OK;
}

// Allocates the bf16 shadow on first prefill use and converts rows [0, len) on `st`.
static int ensure_shadow(spissa_kv_cache *c, hipStream_t st) {
  if (c->kb) return SPISSA_OK;
  const size_t cap = (c->max_seq_len + 63) & ~(size_t)63;
  const size_t elems = cap * c->width();
  ST_TRY(no_capture(st, "the cache's bf16 prefill shadow", 2 * elems * sizeof(bf16)));
  HIP_TRY(hipSetDevice(c->session->device));
  HIP_TRY(hipMalloc(&c->kb, elems * sizeof(bf16)));
  hipError_t e = hipMalloc(&c->vt, elems * sizeof(bf16));
  if (e != hipSuccess) {
    (void)hipFree(c->kb);
    c->kb = nullptr;
    return set_err(SPISSA_ERR_DEVICE, "hipMalloc of the bf16 shadow failed: %s", hipGetErrorString(e));
  }
  c->shadow_cap = cap;
  return shadow_update(c, 0, c->len, st);
}

static int kv_validate_append(const spissa_kv_cache *c, size_t keys_len, size_t values_len,
                              size_t token_count, bool check_lens, size_t *n_out, size_t *new_len) {
  // rotary.rs:227-251, in the same order.
  if (token_count == 0)
    return set_err(SPISSA_ERR_SHAPE, "KV cache append token_count must be greater than zero");
  size_t n;
  if (mul_ovf(token_count, c->width(), &n)) return set_err(SPISSA_ERR_SHAPE, "KV append length overflow");
  if (check_lens && (keys_len != n || values_len != n))
    return set_err(SPISSA_ERR_SHAPE, "KV append shape mismatch: expected %zu, got keys=%zu, values=%zu", n,
                   keys_len, values_len);
  size_t nl;
  if (__builtin_add_overflow(c->len, token_count, &nl)) return set_err(SPISSA_ERR_SHAPE, "KV cache length overflow");
  if (nl > c->max_seq_len)
    return set_err(SPISSA_ERR_SHAPE, "KV cache capacity exceeded: append would set len %zu, max_seq_len %zu",
                   nl, c->max_seq_len);
  *n_out = n;
  *new_len = nl;
  return SPISSA_OK;
}

extern "C" int spissa_kv_cache_append(spissa_kv_cache *c, const float *keys, size_t keys_len,
                                      const float *values, size_t values_len, size_t token_count) {
  GUARD_BEGIN
  if (!c) return set_err(SPISSA_ERR_ARGUMENT, "cache is null");
  size_t n, nl;
  ST_TRY(kv_validate_append(c, keys_len, values_len, token_count, true, &n, &nl));
  if (!keys || !values) return set_err(SPISSA_ERR_ARGUMENT, "keys/values are null");
  spissa_session *s = c->session;
  HIP_TRY(hipSetDevice(s->device));
  const size_t off = c->len * c->width();
  ST_TRY(h2d(s, c->keys + off, keys, n * sizeof(float)));
  ST_TRY(h2d(s, c->values + off, values, n * sizeof(float)));
  ST_TRY(shadow_update(c, c->len, token_count, s->stream));
  ST_TRY(sync_stream(s));
  c->len = nl;
  return SPISSA_OK;
  GUARD_END
}

extern "C" int spissa_kv_cache_append_device(spissa_kv_cache *c, const float *d_keys,
                                             const float *d_values, size_t token_count) {
  GUARD_BEGIN
  if (!c) return set_err(SPISSA_ERR_ARGUMENT, "cache is null");
  size_t n, nl;
  ST_TRY(kv_validate_append(c, 0, 0, token_count, false, &n, &nl));
  if (!d_keys || !d_values) return set_err(SPISSA_ERR_ARGUMENT, "keys/values are null");
  spissa_session *s = c->session;
  HIP_TRY(hipSetDevice(s->device));
  const size_t off = c->len * c->width();
  HIP_TRY(hipMemcpyAsync(c->keys + off, d_keys, n * sizeof(float), hipMemcpyDeviceToDevice, s->stream));
  HIP_TRY(hipMemcpyAsync(c->values + off, d_values, n * sizeof(float), hipMemcpyDeviceToDevice, s->stream));
  ST_TRY(shadow_update(c, c->len, token_count, s->stream));
  c->len = nl;
  return SPISSA_OK;
  GUARD_END
}

extern "C" void spissa_kv_cache_clear(spissa_kv_cache *c) {
  if (c) c->len = 0;
}

extern "C" int spissa_kv_cache_truncate(spissa_kv_cache *c, size_t len) {
  if (!c) return set_err(SPISSA_ERR_ARGUMENT, "cache is null");
  // rotary.rs:264-278
  if (len > c->len) return set_err(SPISSA_ERR_SHAPE, "KV cache truncate cannot grow from %zu to %zu", c->len, len);
  size_t v;
  if (mul_ovf(len, c->width(), &v)) return set_err(SPISSA_ERR_SHAPE, "KV truncate length overflow");
  c->len = len;
  return SPISSA_OK;
}

extern "C" size_t spissa_kv_cache_len(const spissa_kv_cache *c) { return c ? c->len : 0; }
extern "C" int spissa_kv_cache_is_empty(const spissa_kv_cache *c) { return c ? c->len == 0 : 1; }
extern "C" size_t spissa_kv_cache_max_seq_len(const spissa_kv_cache *c) { return c ? c->max_seq_len : 0; }
extern "C" size_t spissa_kv_cache_num_heads(const spissa_kv_cache *c) { return c ? c->num_heads : 0; }
extern "C" size_t spissa_kv_cache_head_dim(const spissa_kv_cache *c) { return c ? c->head_dim : 0; }

// rotary.rs:280-285 (saturating multiply)
extern "C" size_t spissa_kv_cache_resident_bytes(const spissa_kv_cache *c) {
  if (!c) return 0;
  size_t r;
  if (mul_ovf(c->len, c->width(), &r) || mul_ovf(r, 2, &r) || mul_ovf(r, sizeof(float), &r))
    return (size_t)-1;
  return r;
}

static int kv_read(const spissa_kv_cache *c, const float *src, float *dst, size_t dst_len) {
  if (!c) return set_err(SPISSA_ERR_ARGUMENT, "cache is null");
  const size_t n = c->len * c->width();
  if (dst_len < n) return set_err(SPISSA_ERR_SHAPE, "destination holds %zu floats, cache has %zu", dst_len, n);
  if (n == 0) return SPISSA_OK;
  if (!dst) return set_err(SPISSA_ERR_ARGUMENT, "dst is null");
  spissa_session *s = c->session;
  HIP_TRY(hipSetDevice(s->device));
  ST_TRY(d2h(s, dst, src, n * sizeof(float)));
  return sync_stream(s);
}

extern "C" int spissa_kv_cache_read_keys(const spissa_kv_cache *c, float *dst, size_t dst_len) {
  GUARD_BEGIN
  return kv_read(c, c ? c->keys : nullptr, dst, dst_len);
  GUARD_END
}
extern "C" int spissa_kv_cache_read_values(const spissa_kv_cache *c, float *dst, size_t dst_len) {
  GUARD_BEGIN
  return kv_read(c, c ? c->values : nullptr, dst, dst_len);
  GUARD_END
}
extern "C" const float *spissa_kv_cache_device_keys(const spissa_kv_cache *c) { return c ? c->keys : nullptr; }
extern "C" const float *spissa_kv_cache_device_values(const spissa_kv_cache *c) { return c ? c->values : nullptr; }

extern "C" int spissa_kv_cache_clone(const spissa_kv_cache *c, spissa_kv_cache **out) {
  GUARD_BEGIN
  if (!c || !out) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  spissa_kv_cache *n = nullptr;
  ST_TRY(kv_new_impl(c->session, c->num_heads, c->head_dim, c->max_seq_len, &n));
  spissa_session *s = c->session;
  const size_t bytes = c->len * c->width() * sizeof(float);
  hipError_t e = hipSuccess;
  if (bytes) {
    e = hipMemcpyAsync(n->keys, c->keys, bytes, hipMemcpyDeviceToDevice, s->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(n->values, c->values, bytes, hipMemcpyDeviceToDevice, s->stream);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
  if (e != hipSuccess) {
    spissa_kv_cache_free(n);
    return set_err(SPISSA_ERR_DEVICE, "clone copy failed: %s", hipGetErrorString(e));
  }
  n->len = c->len;
  *out = n;
  return SPISSA_OK;
  GUARD_END
}

// ------------------------------------------------------------------------
// RoPE (rotary.rs:6-193)
// ------------------------------------------------------------------------
namespace {

#pragma clang fp contract(off)
// rotary.rs:454-465 rotary_angle -> cos/sin (llama and gpt-neox kinds).
inline void llama_cos_sin(size_t abs_pos, float inv_freq, float *c, float *s) {
  const float angle = (float)abs_pos * inv_freq;
  *c = cosf(angle);
  *s = sinf(angle);
}
inline float llama_inv_freq(size_t pair, size_t rotary_dim, float base, float scale) {
  const float exponent = (float)(2 * pair) / (float)rotary_dim;
  return 1.0f / (powf(base, exponent) * scale);
}
// rotary.rs:168 and 188-193 (gemma kind).
inline float gemma_inv_freq(size_t pair, size_t rotary_dim, float base) {
  const float exponent = (float)(2 * pair) / (float)rotary_dim;
  return 1.0f / powf(base, exponent);
}
inline void gemma_cos_sin(size_t abs_pos, float divisor, float inv_freq, float *c, float *s) {
  const float scaled_pos = (float)abs_pos / divisor;
  const float angle = scaled_pos * inv_freq;
  *c = cosf(angle);
  *s = sinf(angle);
}
#pragma clang fp contract(on)

// Fills cos/sin [n_pos][half] for absolute positions first .. first + n_pos.
void fill_table(int kind, size_t rotary_dim, size_t half, float base, float divisor,
                const float *freq_scale, size_t freq_scale_len, size_t first, size_t n_pos,
                float *cos_out, float *sin_out) {
  std::vector<float> inv(half);
  for (size_t p = 0; p < half; ++p) {
    if (kind == SPISSA_ROPE_GEMMA) {
      inv[p] = gemma_inv_freq(p, rotary_dim, base);
    } else {
      const float scale =
          (kind == SPISSA_ROPE_LLAMA && freq_scale && p < freq_scale_len) ? freq_scale[p] : 1.0f;
      inv[p] = llama_inv_freq(p, rotary_dim, base, scale);
    }
  }
  auto work = [&](size_t r0, size_t r1) {
    for (size_t r = r0; r < r1; ++r)
      for (size_t p = 0; p < half; ++p) {
        float c, s;
        if (kind == SPISSA_ROPE_GEMMA)
          gemma_cos_sin(first + r, divisor, inv[p], &c, &s);
        else
          llama_cos_sin(first + r, inv[p], &c, &s);
        cos_out[r * half + p] = c;
        sin_out[r * half + p] = s;
      }
  };
  const size_t total = n_pos * half;
  unsigned nt = total > (1u << 16) ? std::min(16u, std::max(1u, std::thread::hardware_concurrency())) : 1u;
  if (nt <= 1) {
    work(0, n_pos);
    return;
  }
  std::vector<std::thread> ts;
  size_t per = (n_pos + nt - 1) / nt;
  for (unsigned t = 0; t < nt; ++t) {
    size_t a = t * per, b = std::min(n_pos, a + per);
    if (a < b) ts.emplace_back(work, a, b);
  }
  for (auto &t : ts) t.join();
}

// Runs RoPE on host q/k through the device kernel with a per-call table.
int rope_dropin(int kind, float *q, size_t q_len, float *k, size_t k_len, size_t qh, size_t kh,
                const spissa_rotary_config *cfg, float divisor, const float *fs, size_t fs_len) {
  spissa_session *s = nullptr;
  ST_TRY(spissa_default_session(&s));
  const size_t half = cfg->rotary_dim / 2;
  const size_t S = cfg->seq_len;
  if (S == 0 || half == 0 || (q_len == 0 && k_len == 0)) return SPISSA_OK;
  std::vector<float> cs(S * half), sn(S * half);
  fill_table(kind, cfg->rotary_dim, half, cfg->base, divisor, fs, fs_len, cfg->position_offset, S,
             cs.data(), sn.data());
  float *r[4];
  ST_TRY(io_regions(s, {q_len, k_len, S * half, S * half}, r));
  HIP_TRY(hipSetDevice(s->device));
  ST_TRY(h2d(s, r[0], q, q_len * sizeof(float)));
  ST_TRY(h2d(s, r[1], k, k_len * sizeof(float)));
  ST_TRY(h2d(s, r[2], cs.data(), cs.size() * sizeof(float)));
  ST_TRY(h2d(s, r[3], sn.data(), sn.size() * sizeof(float)));
  HIP_TRY(launch_rope_apply(s->stream, r[2], r[3], half, r[0], r[1], S, qh, kh, cfg->head_dim, half));
  ST_TRY(d2h(s, q, r[0], q_len * sizeof(float)));
  ST_TRY(d2h(s, k, r[1], k_len * sizeof(float)));
  return sync_stream(s);
}

// The reference indexes past the head row when 2*(rotary_dim/2) > head_dim
// (a slice panic, or a write into the next head); this ABI reports Shape.
int guard_half(const spissa_rotary_config *cfg) {
  if (cfg->seq_len > 0 && 2 * (cfg->rotary_dim / 2) > cfg->head_dim)
    return set_err(SPISSA_ERR_SHAPE, "rotary_dim %zu exceeds head_dim %zu", cfg->rotary_dim, cfg->head_dim);
  return SPISSA_OK;
}

}  // namespace

extern "C" int spissa_gpt_neox_rotary_dim(size_t head_dim, float rotary_pct, size_t *out) {
  // rotary.rs:17-38
  if (!out) return set_err(SPISSA_ERR_ARGUMENT, "out is null");
  if (head_dim == 0) return set_err(SPISSA_ERR_SHAPE, "head_dim must be greater than zero");
  if (!std::isfinite(rotary_pct) || rotary_pct <= 0.0f || rotary_pct > 1.0f)
    return set_err(SPISSA_ERR_INVALID_TENSOR_DATA, "rotary_pct must be finite and in (0, 1], got %g", rotary_pct);
  const float prod = (float)head_dim * rotary_pct;
  size_t dim = (size_t)prod;
  if (dim % 2 != 0) dim -= 1;
  if (dim == 0)
    return set_err(SPISSA_ERR_SHAPE, "rotary_pct %g produces zero even rotary dim for head_dim %zu", rotary_pct,
                   head_dim);
  *out = dim;
  return SPISSA_OK;
}

extern "C" int spissa_apply_gpt_neox_rotary_inplace(float *q, size_t q_len, float *k, size_t k_len,
                                                    const spissa_rotary_config *cfg) {
  GUARD_BEGIN
  if (!cfg) return set_err(SPISSA_ERR_ARGUMENT, "config is null");
  // rotary.rs:417-452 validate_rotary_inputs
  size_t expected;
  if (mul_ovf(cfg->seq_len, cfg->num_heads, &expected) || mul_ovf(expected, cfg->head_dim, &expected))
    return set_err(SPISSA_ERR_SHAPE, "rotary input length overflow");
  if (q_len != expected || k_len != expected)
    return set_err(SPISSA_ERR_SHAPE, "rotary Q/K shape mismatch: expected %zu, got q=%zu, k=%zu", expected, q_len,
                   k_len);
  if (cfg->seq_len == 0 || cfg->num_heads == 0 || cfg->head_dim == 0)
    return set_err(SPISSA_ERR_SHAPE, "rotary dimensions must be non-zero, got seq_len=%zu, num_heads=%zu, head_dim=%zu",
                   cfg->seq_len, cfg->num_heads, cfg->head_dim);
  if (cfg->rotary_dim == 0 || cfg->rotary_dim > cfg->head_dim || cfg->rotary_dim % 2 != 0)
    return set_err(SPISSA_ERR_SHAPE, "rotary_dim must be even and in 1..=head_dim, got rotary_dim=%zu, head_dim=%zu",
                   cfg->rotary_dim, cfg->head_dim);
  if (!std::isfinite(cfg->base) || cfg->base <= 0.0f)
    return set_err(SPISSA_ERR_INVALID_TENSOR_DATA, "rotary base must be finite and positive, got %g", cfg->base);
  size_t last;
  if (__builtin_add_overflow(cfg->position_offset, cfg->seq_len - 1, &last))
    return set_err(SPISSA_ERR_SHAPE, "rotary absolute position overflow");
  if (!q || !k) return set_err(SPISSA_ERR_ARGUMENT, "q/k are null");
  return rope_dropin(SPISSA_ROPE_NEOX, q, q_len, k, k_len, cfg->num_heads, cfg->num_heads, cfg, 1.0f,
                     nullptr, 0);
  GUARD_END
}

extern "C" int spissa_apply_llama_rotary_inplace(float *q, size_t q_len, float *k, size_t k_len,
                                                 size_t q_heads, size_t k_heads,
                                                 const spissa_rotary_config *cfg,
                                                 const float *freq_scale, size_t freq_scale_len) {
  GUARD_BEGIN
  if (!cfg) return set_err(SPISSA_ERR_ARGUMENT, "config is null");
  // rotary.rs:83-96
  if (q_heads == 0 || k_heads == 0) return set_err(SPISSA_ERR_SHAPE, "heads must be > 0");
  const size_t eq = cfg->seq_len * q_heads * cfg->head_dim;
  const size_t ek = cfg->seq_len * k_heads * cfg->head_dim;
  if (q_len != eq || k_len != ek)
    return set_err(SPISSA_ERR_SHAPE, "rotary shape mismatch: q=%zu, expected=%zu, k=%zu, expected=%zu", q_len, eq,
                   k_len, ek);
  ST_TRY(guard_half(cfg));
  if ((!q && q_len) || (!k && k_len)) return set_err(SPISSA_ERR_ARGUMENT, "q/k are null");
  return rope_dropin(SPISSA_ROPE_LLAMA, q, q_len, k, k_len, q_heads, k_heads, cfg, 1.0f, freq_scale,
                     freq_scale ? freq_scale_len : 0);
  GUARD_END
}

extern "C" int spissa_apply_gemma_rotary_inplace(float *q, size_t q_len, float *k, size_t k_len,
                                                 size_t q_heads, size_t k_heads,
                                                 const spissa_rotary_config *cfg,
                                                 float position_divisor) {
  GUARD_BEGIN
  if (!cfg) return set_err(SPISSA_ERR_ARGUMENT, "config is null");
  // rotary.rs:145-163
  if (q_heads == 0 || k_heads == 0) return set_err(SPISSA_ERR_SHAPE, "heads must be > 0");
  if (!std::isfinite(position_divisor) || position_divisor <= 0.0f)
    return set_err(SPISSA_ERR_INVALID_TENSOR_DATA,
                   "gemma rotary position_divisor must be finite and positive, got %g", position_divisor);
  const size_t eq = cfg->seq_len * q_heads * cfg->head_dim;
  const size_t ek = cfg->seq_len * k_heads * cfg->head_dim;
  if (q_len != eq || k_len != ek)
    return set_err(SPISSA_ERR_SHAPE, "gemma rotary shape mismatch: q=%zu, expected=%zu, k=%zu, expected=%zu", q_len,
                   eq, k_len, ek);
  ST_TRY(guard_half(cfg));
  if ((!q && q_len) || (!k && k_len)) return set_err(SPISSA_ERR_ARGUMENT, "q/k are null");
  return rope_dropin(SPISSA_ROPE_GEMMA, q, q_len, k, k_len, q_heads, k_heads, cfg, position_divisor,
                     nullptr, 0);
  GUARD_END
}

extern "C" int spissa_rope_table_new(spissa_session *s, int kind, size_t rotary_dim, float base,
                                     float position_divisor, const float *freq_scale,
                                     size_t freq_scale_len, size_t max_positions,
                                     spissa_rope_table **out) {
  GUARD_BEGIN
  if (!s || !out) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  *out = nullptr;
  if (kind != SPISSA_ROPE_LLAMA && kind != SPISSA_ROPE_GEMMA && kind != SPISSA_ROPE_NEOX)
    return set_err(SPISSA_ERR_ARGUMENT, "unknown rope kind %d", kind);
  if (rotary_dim < 2 || max_positions == 0)
    return set_err(SPISSA_ERR_SHAPE, "rope table needs rotary_dim >= 2 and max_positions > 0");
  if (kind == SPISSA_ROPE_NEOX && (rotary_dim % 2 != 0 || !std::isfinite(base) || base <= 0.0f))
    return set_err(base <= 0.0f || !std::isfinite(base) ? SPISSA_ERR_INVALID_TENSOR_DATA : SPISSA_ERR_SHAPE,
                   "invalid gpt-neox rotary parameters");
  if (kind == SPISSA_ROPE_GEMMA && (!std::isfinite(position_divisor) || position_divisor <= 0.0f))
    return set_err(SPISSA_ERR_INVALID_TENSOR_DATA,
                   "gemma rotary position_divisor must be finite and positive, got %g", position_divisor);
  const size_t half = rotary_dim / 2;
  size_t n;
  if (mul_ovf(max_positions, half, &n)) return set_err(SPISSA_ERR_SHAPE, "rope table size overflow");
  std::vector<float> cs(n), sn(n);
  fill_table(kind, rotary_dim, half, base, position_divisor, freq_scale, freq_scale ? freq_scale_len : 0, 0,
             max_positions, cs.data(), sn.data());
  std::unique_ptr<spissa_rope_table> t(new spissa_rope_table());
  t->device = s->device;
  t->kind = kind;
  t->rotary_dim = rotary_dim;
  t->half = half;
  t->max_positions = max_positions;
  HIP_TRY(hipSetDevice(s->device));
  HIP_TRY(hipMalloc(&t->cos, n * sizeof(float)));
  HIP_TRY(hipMalloc(&t->sin, n * sizeof(float)));
  HIP_TRY(hipMemcpy(t->cos, cs.data(), n * sizeof(float), hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(t->sin, sn.data(), n * sizeof(float), hipMemcpyHostToDevice));
  *out = t.release();
  return SPISSA_OK;
  GUARD_END
}

extern "C" void spissa_rope_table_free(spissa_rope_table *t) {
  if (!t) return;
  (void)hipSetDevice(t->device);
  (void)hipDeviceSynchronize();
  if (t->cos) (void)hipFree(t->cos);
  if (t->sin) (void)hipFree(t->sin);
  delete t;
}

static int table_check(const spissa_rope_table *t, size_t seq_len, size_t head_dim, size_t offset) {
  if (2 * t->half > head_dim)
    return set_err(SPISSA_ERR_SHAPE, "rotary_dim %zu exceeds head_dim %zu", t->rotary_dim, head_dim);
  size_t end;
  if (__builtin_add_overflow(offset, seq_len, &end) || end > t->max_positions)
    return set_err(SPISSA_ERR_SHAPE, "positions %zu..%zu exceed the rope table (%zu positions)", offset,
                   offset + seq_len, t->max_positions);
  return SPISSA_OK;
}

extern "C" int spissa_rope_apply_device(spissa_session *s, const spissa_rope_table *t, float *d_q,
                                        float *d_k, size_t seq_len, size_t q_heads, size_t k_heads,
                                        size_t head_dim, size_t position_offset) {
  GUARD_BEGIN
  if (!s || !t) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  if (q_heads == 0 || k_heads == 0) return set_err(SPISSA_ERR_SHAPE, "heads must be > 0");
  ST_TRY(table_check(t, seq_len, head_dim, position_offset));
  HIP_TRY(hipSetDevice(s->device));
  HIP_TRY(launch_rope_apply(s->stream, t->cos + position_offset * t->half, t->sin + position_offset * t->half,
                            t->half, d_q, d_k, seq_len, q_heads, k_heads, head_dim, t->half));
  return SPISSA_OK;
  GUARD_END
}

// ------------------------------------------------------------------------
// RMSNorm and the Gemma prologue
// ------------------------------------------------------------------------
extern "C" int spissa_rms_norm(const float *x, size_t x_len, const float *weight, size_t weight_len,
                               size_t rows, size_t cols, float eps, float *out, size_t out_len) {
  GUARD_BEGIN
  // ops.rs:160-166
  if (x_len != rows * cols || weight_len != cols)
    return set_err(SPISSA_ERR_SHAPE, "rms_norm shape mismatch: x=%zu, rows=%zu, cols=%zu, weight=%zu", x_len, rows,
                   cols, weight_len);
  if (out_len != x_len) return set_err(SPISSA_ERR_SHAPE, "rms_norm output holds %zu floats, need %zu", out_len, x_len);
  if (x_len == 0) return SPISSA_OK;
  if (!x || !weight || !out) return set_err(SPISSA_ERR_ARGUMENT, "null buffer");
  spissa_session *s = nullptr;
  ST_TRY(spissa_default_session(&s));
  float *r[3];
  ST_TRY(io_regions(s, {x_len, cols, x_len}, r));
  HIP_TRY(hipSetDevice(s->device));
  ST_TRY(h2d(s, r[0], x, x_len * sizeof(float)));
  ST_TRY(h2d(s, r[1], weight, cols * sizeof(float)));
  HIP_TRY(launch_rms_norm(s->stream, r[0], r[1], rows, cols, eps, r[2]));
  ST_TRY(d2h(s, out, r[2], x_len * sizeof(float)));
  return sync_stream(s);
  GUARD_END
}

extern "C" int spissa_rms_norm_device(spissa_session *s, const float *d_x, const float *d_weight, size_t rows,
                                      size_t cols, float eps, float *d_out) {
  GUARD_BEGIN
  if (!s) return set_err(SPISSA_ERR_ARGUMENT, "session is null");
  HIP_TRY(hipSetDevice(s->device));
  HIP_TRY(launch_rms_norm(s->stream, d_x, d_weight, rows, cols, eps, d_out));
  return SPISSA_OK;
  GUARD_END
}

extern "C" int spissa_is_global_layer(size_t layer_idx, size_t pattern) {
  // models/gemma/model.rs:46-51
  if (pattern <= 1) return 1;
  return (layer_idx + 1) % pattern == 0;
}

extern "C" int spissa_gemma_qk_prologue_device(spissa_session *s, const spissa_rope_table *t, float *d_q,
                                               float *d_k, size_t seq_len, size_t q_heads, size_t kv_heads,
                                               size_t head_dim, const float *d_q_norm, const float *d_k_norm,
                                               float eps, size_t position_offset, float q_prescale) {
  GUARD_BEGIN
  if (!s || !t) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  if (t->kind != SPISSA_ROPE_GEMMA) return set_err(SPISSA_ERR_ARGUMENT, "the gemma prologue needs a gemma rope table");
  if (q_heads == 0 || kv_heads == 0 || head_dim == 0) return set_err(SPISSA_ERR_SHAPE, "dimensions must be > 0");
  ST_TRY(table_check(t, seq_len, head_dim, position_offset));
  HIP_TRY(hipSetDevice(s->device));
  HIP_TRY(launch_gemma_prologue(s->stream, t->cos + position_offset * t->half, t->sin + position_offset * t->half,
                                t->half, d_q, d_k, seq_len, q_heads, kv_heads, head_dim, t->half, d_q_norm,
                                d_k_norm, eps, q_prescale));
  return SPISSA_OK;
  GUARD_END
}

// ------------------------------------------------------------------------
// Attention (rotary.rs:335-415)
// ------------------------------------------------------------------------
static int validate_attention(size_t q_len, size_t k_len, size_t v_len, const spissa_kv_cache *cache,
                              const spissa_kv_attention_config *c, bool check_lens) {
  // rotary.rs:483-547, same order.
  if (c->query_len == 0 || c->num_heads == 0 || c->kv_heads == 0 || c->head_dim == 0)
    return set_err(SPISSA_ERR_SHAPE,
                   "KV attention dimensions must be non-zero, got query_len=%zu, num_heads=%zu, kv_heads=%zu, "
                   "head_dim=%zu",
                   c->query_len, c->num_heads, c->kv_heads, c->head_dim);
  if (c->num_heads % c->kv_heads != 0)
    return set_err(SPISSA_ERR_SHAPE, "query heads %zu must be a multiple of key/value heads %zu", c->num_heads,
                   c->kv_heads);
  size_t eq, ekv;
  if (mul_ovf(c->query_len, c->num_heads, &eq) || mul_ovf(eq, c->head_dim, &eq))
    return set_err(SPISSA_ERR_SHAPE, "KV attention current length overflow");
  if (mul_ovf(c->query_len, c->kv_heads, &ekv) || mul_ovf(ekv, c->head_dim, &ekv))
    return set_err(SPISSA_ERR_SHAPE, "KV attention current length overflow");
  if (check_lens && (q_len != eq || k_len != ekv || v_len != ekv))
    return set_err(SPISSA_ERR_SHAPE, "KV attention shape mismatch: expected q=%zu, k/v=%zu, got q=%zu, k=%zu, v=%zu",
                   eq, ekv, q_len, k_len, v_len);
  if (cache && (cache->num_heads != c->kv_heads || cache->head_dim != c->head_dim))
    return set_err(SPISSA_ERR_SHAPE, "KV cache shape mismatch: cache heads/dim=%zu/%zu, attention kv_heads/dim=%zu/%zu",
                   cache->num_heads, cache->head_dim, c->kv_heads, c->head_dim);
  size_t past = cache ? cache->len : 0, key_len;
  if (__builtin_add_overflow(past, c->query_len, &key_len)) return set_err(SPISSA_ERR_SHAPE, "KV attention key length overflow");
  // Device index arithmetic is 32-bit in the key dimension.
  if (key_len > (size_t)INT32_MAX / 2 || c->num_heads > 65535 || c->window > (size_t)INT32_MAX)
    return set_err(SPISSA_ERR_SHAPE, "attention sizes exceed the device kernels' limits");
  return SPISSA_OK;
}

// The split-K decode kernel addresses a cache buffer with 32-bit byte offsets.
static bool decode_cache_fits(const spissa_kv_cache *c) {
  return !c || (double)c->max_seq_len * c->width() * sizeof(float) < 4294967296.0;
}

static int pick_rb(int R) {
  if (R % 4 == 0) return 4;
  if (R % 3 == 0) return 3;
  if (R % 2 == 0) return 2;
  return 1;
}

// Launch plan of one split-K decode launch over B <= kMaxDecodeBatch
// sequences with past[b] cached tokens each.
struct DecodePlan {
  int RB = 1, HB = 1;    // query heads per block, head blocks per KV head
  int kps = 0;           // cached keys per split
  int max_splits = 0;    // splits of the longest sequence (with the token's own)
  int tok_split = 0;     // the new token has a split of its own
  size_t workgroups = 0; // split-kernel grid
  size_t partial_bytes = 0;
};

// partial_cap: bytes available for the partials (0: unbounded). Returns false
// when even one split per (sequence, KV head, head block) does not fit.
static bool plan_decode(int D, int Hq, int Hkv, size_t window, const int *past, int B, size_t partial_cap,
                        DecodePlan *p) {
  const int R = Hq / Hkv;
  p->RB = pick_rb(R);
  p->HB = R / p->RB;
  int max_keys = 0;
  int keys[kMaxDecodeBatch];  // (B <= kMaxDecodeBatch: one launch's sequences)
  for (int b = 0; b < B; ++b) {
    const int P = past[b];
    const int kstart = window > 0 ? std::max(0, P + 1 - (int)window) : 0;
    const int cached = P - kstart;  // visible cached keys; the new token is handled apart
    max_keys = std::max(max_keys, cached);
    keys[b] = cached;
  }
  const size_t groups = (size_t)B * Hkv * p->HB;
  const size_t entry = (size_t)p->RB * (D + 2) * sizeof(float);
  // The new token gets a split of its own, dispatched first, so that its
  // loads, QK-norm and append run beside the streaming splits -- when the
  // whole grid stays within kDecodeGridWorkgroups (measured: the Gemma decode
  // layers 9-11% faster; past it the token workgroups cost more than they
  // save: batch 16, 640 against 512 workgroups, 205 against 171 us; Llama-3.2-1B
  // at 2048 keys, 520 against 512, 8.4 against 8.1 us) and a fixed partial
  // buffer holds two entries per group. Otherwise split 0 takes it after its
  // cached rows.
  int split_cap = kMaxDecodeSplits;
  p->tok_split = 1;
  if (partial_cap) {
    const size_t fit = partial_cap / (groups * entry);
    if (fit < 1) return false;
    p->tok_split = fit >= 2 ? 1 : 0;
    split_cap = (int)std::min<size_t>(fit, kMaxDecodeSplits);
  }
  p->kps = decode_keys_per_split(D, p->RB, keys, B, (long)Hkv * p->HB, split_cap - p->tok_split);
  const int cached_splits = (max_keys + p->kps - 1) / p->kps;
  if (groups * (size_t)(cached_splits + 1) > (size_t)kDecodeGridWorkgroups) p->tok_split = 0;
  p->max_splits = p->tok_split ? cached_splits + 1 : std::max(1, cached_splits);
  p->workgroups = groups * p->max_splits;
  p->partial_bytes = groups * p->max_splits * entry;
  return true;
}

// Split-K decode over `batch` sequences (one new token each). Optionally fuses
// the RoPE of q/k from `table` (rotate-half over the whole head) and the
// append of the new key and value to each cache; the caller has validated
// capacity when `append` is set. The partials go to the session workspace,
// or, with `fixed` set, to the fixed_bytes at `fixed` (splits are coarsened
// to fit; the caller has checked that one split per group fits).
struct GemmaQkNorm {  // fused QK-norm of the Gemma decode step
  const float *q_norm, *k_norm;
  float eps, q_prescale;
};

static int run_decode(spissa_session *s, const float *d_q, const float *d_k, const float *d_v,
                      const spissa_kv_cache *const *caches, size_t batch, const spissa_kv_attention_config *c,
                      float *d_out, const spissa_rope_table *table, bool append, float *fixed = nullptr,
                      size_t fixed_bytes = 0, const GemmaQkNorm *norm = nullptr) {
  const int D = (int)c->head_dim, Hq = (int)c->num_heads, Hkv = (int)c->kv_heads;
  const int R = Hq / Hkv;
  for (size_t b0 = 0; b0 < batch; b0 += kMaxDecodeBatch) {
    const int B = (int)std::min<size_t>(kMaxDecodeBatch, batch - b0);
    DecodeArgs a;
    memset(&a, 0, sizeof a);
    int past[kMaxDecodeBatch];
    for (int b = 0; b < B; ++b) {
      const spissa_kv_cache *cb = caches ? caches[b0 + b] : nullptr;
      const int P = cb ? (int)cb->len : 0;
      past[b] = P;
      a.seq[b].k = cb ? cb->keys : nullptr;
      a.seq[b].v = cb ? cb->values : nullptr;
      a.seq[b].past = P;
      if (append) {
        a.app_k[b] = cb->keys + (size_t)P * cb->width();
        a.app_v[b] = cb->values + (size_t)P * cb->width();
        a.app_kb[b] = cb->kb;
        a.app_vt[b] = cb->vt;
        a.app_cap[b] = (long)cb->shadow_cap;
      }
    }
    DecodePlan plan;
    if (!plan_decode(D, Hq, Hkv, c->window, past, B, fixed ? fixed_bytes : 0, &plan))
      return set_err(SPISSA_ERR_SHAPE, "decode partials of %d sequences x %d heads exceed %zu bytes", B, Hq,
                     fixed_bytes);
    const int RB = plan.RB, HB = plan.HB, kps = plan.kps, max_splits = plan.max_splits;
    if (!fixed) ST_TRY(ensure_buf(s, s->partial, plan.partial_bytes));
    a.q = const_cast<float *>(d_q) + b0 * (size_t)Hq * D;
    a.cur_k = const_cast<float *>(d_k) + b0 * (size_t)Hkv * D;
    a.cur_v = d_v + b0 * (size_t)Hkv * D;
    a.out = d_out + b0 * (size_t)Hq * D;
    a.partial = fixed ? fixed : (float *)s->partial.p;
    a.err = s->d_err;
    a.rope_cos = table ? table->cos : nullptr;
    a.rope_sin = table ? table->sin : nullptr;
    a.do_append = append ? 1 : 0;
    if (norm) {
      a.q_norm = norm->q_norm;
      a.k_norm = norm->k_norm;
      a.norm_eps = norm->eps;
      a.q_prescale = norm->q_prescale;
    }
    a.B = B;
    a.Hq = Hq;
    a.Hkv = Hkv;
    a.R = R;
    a.HB = HB;
    a.window = (int)c->window;
    a.kps = kps;
    a.max_splits = max_splits;
    a.tok_split = plan.tok_split;
    a.qscale = (1.0f / sqrtf((float)D)) * 1.4426950408889634f;
    HIP_TRY(launch_decode(s->stream, a, D, RB));
  }
  return SPISSA_OK;
}

static int run_generic(spissa_session *s, const float *d_q, const float *d_k, const float *d_v,
                       const spissa_kv_cache *cache, const spissa_kv_attention_config *c, float *d_out) {
  GenericArgs g;
  g.q = d_q;
  g.cur_k = d_k;
  g.cur_v = d_v;
  g.cache_k = cache ? cache->keys : nullptr;
  g.cache_v = cache ? cache->values : nullptr;
  g.out = d_out;
  g.err = s->d_err;
  g.S = (int)c->query_len;
  g.P = cache ? (int)cache->len : 0;
  g.Hq = (int)c->num_heads;
  g.Hkv = (int)c->kv_heads;
  g.D = (int)c->head_dim;
  g.R = g.Hq / g.Hkv;
  g.causal = c->causal ? 1 : 0;
  g.window = (int)c->window;
  g.scale = 1.0f / sqrtf((float)c->head_dim);
  if (g.D > 1024) return set_err(SPISSA_ERR_SHAPE, "head_dim %d exceeds the f32 kernel's limit of 1024", g.D);
  HIP_TRY(launch_generic(s->stream, g));
  return SPISSA_OK;
}

// Launch plan of one bf16 prefill call (S > 1 queries over P cached keys):
// staging geometry, key splits and the head_dim-256 O split, set in `a`
// (whose P, S, Hq, Hkv, R, causal and window are filled in).
struct PrefillPlan {
  int P8 = 0;              // keys below come from the cache's bf16 shadow
  size_t cap_stage = 0;    // staging rows per KV head (tile-aligned)
  size_t stage_bytes = 0;  // bf16 K and V^T staging
  size_t ppart_bytes = 0;  // key-split partials (0: no splits)
  long tiles = 0;          // most key tiles of one unsplit workgroup
  size_t workgroups = 0;
};

static void plan_prefill(PrefillArgs &a, int D, int cus, PrefillPlan *p) {
  const int P = a.P, S = a.S;
  // Keys [0, P8) are read from the cache's bf16 shadow, keys [P8, P+S) from
  // the staging buffer; P8 is tile-aligned so no key tile straddles the two.
  p->P8 = P & ~(kPrefillTileAlign - 1);
  p->cap_stage = (((size_t)P + S + kPrefillTileAlign - 1) & ~(size_t)(kPrefillTileAlign - 1)) - p->P8;
  p->stage_bytes = 2 * (size_t)a.Hkv * p->cap_stage * D * sizeof(bf16);
  a.P8 = p->P8;
  a.cap_stage = (long)p->cap_stage;
  a.splits = 1;
  a.tps = 0;
  const long slots = (long)cus * prefill_wgs_per_cu(a, D);
  a.ksp = 1;
  a.ksp = prefill_wave_pairs(a, D, slots);
  // Key splits when the unsplit grid cannot fill the GPU (short chunks over
  // long caches, few heads): enough splits for one round of workgroup slots,
  // each covering at least four key tiles of its workgroup's range (eight
  // for windowed head_dim-256 layers: Gemma-3-4B's W1024 chunk of 128 on
  // 16384 keys measured 23.4 us with 4 splits against 25.1 us with 9). The
  // splits cover the widest tile range any workgroup has, so every
  // workgroup's keys are covered. Head_dim-64/128 chunks (at least as many
  // cached keys as queries, so every block sees a similar range) aim at three
  // quarters of a round: Llama-3.2-3B chunks of 256 on 8192 keys / 512 on
  // 4096 / 64 on 8192 measured 55.5 / 58.2 / 34.2 us at 384 workgroups
  // against 66.8 / 66.8 / 38.6 us at a full round.
  // Causal head_dim-64/128 prompts (fewer cached keys than queries) run
  // unsplit unless their grid fills at most a quarter of the slots and their
  // longest query blocks visit at least 32 tiles: their partials are as large
  // as the output, and writing and merging them cost more than short chains
  // or a few idle slots save (reference-order call per layer: Llama-3.2-1B
  // 1024-token prompt 33.2 us with 2 splits against 24.2 unsplit, 512 tokens
  // 19.2 against 15.5; Llama-3.2-3B 512 / 1024 / 2048 tokens 27.9 / 40.1 /
  // 67.9 split against 21.9 / 33.7 / 57.9 unsplit). Long chains on small
  // grids still split (one GPU's share of Llama-3.2-3B's heads, 96
  // workgroups of 64 tiles: 45.2 us with 6 splits against 77.2 unsplit; 4
  // query heads on 1 KV head, 2048 tokens at head_dim 64, 128 paired
  // workgroups: 24.1 with 4 splits against 26.5).
  const long base = prefill_base_workgroups(a, D);
  p->tiles = prefill_max_tile_span(a, D);
  const bool full_prompt = a.causal && a.P < a.S && D < 256 && (4 * base > slots || p->tiles < 32);
  if (base < slots && !full_prompt) {
    const long min_tiles = D >= 256 && a.window > 0 ? 8 : 4;
    // (Head_dim-256 causal prompts aim at one and a half rounds: the upper
    // splits of the short blocks are empty and exit at once, so the grid's
    // real work still fits about one round while the longest chain shrinks.
    // Gemma-3-1B's global 4096-token layer, 2 / 3 / 4 splits: 86.8 / 74.5-77.2
    // / 102.2 us.)
    const long target = a.P >= a.S && D < 256          ? slots * 3 / 4
                        : a.causal && a.P < a.S && D >= 256 ? slots * 3 / 2
                                                            : slots;
    const long want = std::min(std::min((target + base - 1) / base, p->tiles / min_tiles), (long)D);
    if (want >= 2) {  // (at most head_dim splits: the measured useful range)
      a.tps = (int)((p->tiles + want - 1) / want);
      a.splits = (int)((p->tiles + a.tps - 1) / a.tps);
      p->ppart_bytes = (size_t)a.splits * S * a.Hq * (D + 2) * sizeof(float);
    }
  }
  // Windowed head_dim-256 layers with at least one workgroup per two CUs run
  // unsplit: the key-split combine costs more than the CUs left idle
  // (measured on Gemma-3-1B's W512 layer: 42.8 against 46.6 us).
  if (D >= 256 && a.window > 0 && base * 2 >= cus) {
    a.splits = 1;
    a.tps = 0;
    p->ppart_bytes = 0;
  }
  a.xcd_group = prefill_use_xcd_group(a, D);
  const int wgq = prefill_wg_queries(a, D);
  p->workgroups = (size_t)prefill_grid_workgroups((S + wgq - 1) / wgq, a.R / prefill_wg_heads(a, D), a.Hkv, a.splits,
                                                  a.xcd_group);
}

static void prefill_args_base(PrefillArgs &a, const spissa_kv_attention_config *c, int P) {
  memset(&a, 0, sizeof a);
  a.P = P;
  a.S = (int)c->query_len;
  a.Hq = (int)c->num_heads;
  a.Hkv = (int)c->kv_heads;
  a.R = a.Hq / a.Hkv;
  a.causal = c->causal ? 1 : 0;
  a.window = (int)c->window;
  a.qk_scale_log2 = (1.0f / sqrtf((float)c->head_dim)) * 1.4426950408889634f;
}

static int run_prefill(spissa_session *s, const float *d_q, const float *d_k, const float *d_v,
                       spissa_kv_cache *cache, const spissa_kv_attention_config *c, float *d_out) {
  const int D = (int)c->head_dim, Hkv = (int)c->kv_heads;
  const int P = cache ? (int)cache->len : 0;
  const int S = (int)c->query_len;
  PrefillArgs a;
  prefill_args_base(a, c, P);
  PrefillPlan plan;
  plan_prefill(a, D, s->cus, &plan);
  const int P8 = plan.P8;
  const size_t cap_stage = plan.cap_stage;
  if (cache && P8 > 0) ST_TRY(ensure_shadow(cache, s->stream));
  ST_TRY(ensure_buf(s, s->stage, plan.stage_bytes));
  if (plan.ppart_bytes) ST_TRY(ensure_buf(s, s->ppart, plan.ppart_bytes));
  bf16 *kb_stage = (bf16 *)s->stage.p;
  bf16 *vt_stage = kb_stage + (size_t)Hkv * cap_stage * D;
  const size_t w = (size_t)Hkv * D;
  const int tail = P - P8;  // cached rows re-staged so the staging buffer starts tile-aligned
  if (tail > 0)
    HIP_TRY(launch_stage_bf16(s->stream, cache->keys + (size_t)P8 * w, cache->values + (size_t)P8 * w, tail, tail,
                              Hkv, D, kb_stage, vt_stage, 0, cap_stage));
  HIP_TRY(launch_stage_bf16(s->stream, d_k, d_v, S, cap_stage - tail, Hkv, D, kb_stage, vt_stage, tail, cap_stage));
  a.q = d_q;
  a.out = d_out;
  a.kb_cache = cache ? cache->kb : nullptr;
  a.vt_cache = cache ? cache->vt : nullptr;
  a.kb_stage = kb_stage;
  a.vt_stage = vt_stage;
  a.cap_cache = cache ? (long)cache->shadow_cap : 0;
  a.err = s->d_err;
  if (a.splits > 1) {
    const size_t rows = (size_t)a.splits * S * a.Hq;
    a.part_o = (float *)s->ppart.p;
    a.part_ml = a.part_o + rows * D;
  }
  HIP_TRY(launch_prefill(s->stream, a, D));
  HIP_TRY(launch_prefill_combine(s->stream, a, D));
  return SPISSA_OK;
}

static int attention_device_impl(spissa_session *s, const float *d_q, const float *d_k, const float *d_v,
                                 const spissa_kv_cache *cache, const spissa_kv_attention_config *c, float *d_out) {
  HIP_TRY(hipSetDevice(s->device));
  const int D = (int)c->head_dim;
  const int R = (int)(c->num_heads / c->kv_heads);
  if (c->query_len == 1 && decode_supported(D, R) && decode_cache_fits(cache))
    return run_decode(s, d_q, d_k, d_v, &cache, 1, c, d_out, nullptr, false);
  if (c->query_len > 1 && s->prefill_precision == SPISSA_PREFILL_BF16 && prefill_supported(D))
    return run_prefill(s, d_q, d_k, d_v, const_cast<spissa_kv_cache *>(cache), c, d_out);
  return run_generic(s, d_q, d_k, d_v, cache, c, d_out);
}

extern "C" int spissa_attention_device(spissa_session *s, const float *d_q, const float *d_k, const float *d_v,
                                       const spissa_kv_cache *cache, const spissa_kv_attention_config *cfg,
                                       float *d_out) {
  GUARD_BEGIN
  if (!s || !cfg) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  ST_TRY(validate_attention(0, 0, 0, cache, cfg, false));
  if (cache && cache->session->device != s->device)
    return set_err(SPISSA_ERR_ARGUMENT, "cache lives on device %d, session on %d", cache->session->device, s->device);
  return attention_device_impl(s, d_q, d_k, d_v, cache, cfg, d_out);
  GUARD_END
}

extern "C" int spissa_attention_decode_batch_device(spissa_session *s, const float *d_q, const float *d_k,
                                                    const float *d_v, const spissa_kv_cache *const *caches,
                                                    size_t batch, const spissa_kv_attention_config *cfg,
                                                    float *d_out) {
  GUARD_BEGIN
  if (!s || !cfg) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  if (cfg->query_len != 1) return set_err(SPISSA_ERR_SHAPE, "batched decode needs query_len == 1, got %zu", cfg->query_len);
  for (size_t b = 0; b < batch; ++b) ST_TRY(validate_attention(0, 0, 0, caches ? caches[b] : nullptr, cfg, false));
  if (batch == 0) return SPISSA_OK;
  HIP_TRY(hipSetDevice(s->device));
  const int D = (int)cfg->head_dim;
  const int R = (int)(cfg->num_heads / cfg->kv_heads);
  bool fits = true;
  for (size_t b = 0; b < batch; ++b) fits = fits && decode_cache_fits(caches ? caches[b] : nullptr);
  if (decode_supported(D, R) && fits) return run_decode(s, d_q, d_k, d_v, caches, batch, cfg, d_out, nullptr, false);
  for (size_t b = 0; b < batch; ++b) {
    const size_t qo = b * cfg->num_heads * cfg->head_dim, ko = b * cfg->kv_heads * cfg->head_dim;
    ST_TRY(run_generic(s, d_q + qo, d_k + ko, d_v + ko, caches ? caches[b] : nullptr, cfg, d_out + qo));
  }
  return SPISSA_OK;
  GUARD_END
}

// Every check of a fused decode step, before anything runs.
static int validate_decode_step(spissa_session *s, const spissa_rope_table *table, spissa_kv_cache *const *caches,
                                size_t batch, const spissa_kv_attention_config *cfg) {
  if (!s || !cfg || !caches) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  if (cfg->query_len != 1) return set_err(SPISSA_ERR_SHAPE, "a decode step needs query_len == 1, got %zu", cfg->query_len);
  for (size_t b = 0; b < batch; ++b) {
    if (!caches[b]) return set_err(SPISSA_ERR_ARGUMENT, "cache %zu is null", b);
    ST_TRY(validate_attention(0, 0, 0, caches[b], cfg, false));
    size_t n, nl;  // rotary.rs:227-251: the append must fit before anything runs
    ST_TRY(kv_validate_append(caches[b], 0, 0, 1, false, &n, &nl));
    if (caches[b]->session->device != s->device)
      return set_err(SPISSA_ERR_ARGUMENT, "cache %zu lives on another device", b);
    if (!decode_cache_fits(caches[b]))
      return set_err(SPISSA_ERR_SHAPE, "cache %zu exceeds the fused decode step's 4 GiB per-buffer limit", b);
  }
  // Each sequence appends one row at its own length: a cache listed twice
  // would have both tokens written to the same row.
  std::vector<const spissa_kv_cache *> seen(caches, caches + batch);
  std::sort(seen.begin(), seen.end());
  if (std::adjacent_find(seen.begin(), seen.end()) != seen.end())
    return set_err(SPISSA_ERR_ARGUMENT, "a cache appears more than once in one decode step");
  const int D = (int)cfg->head_dim;
  if (!decode_supported(D, (int)(cfg->num_heads / cfg->kv_heads)))
    return set_err(SPISSA_ERR_SHAPE, "the fused decode step supports head_dim 64, 128 and 256, got %d", D);
  if (table) {
    if (table->kind == SPISSA_ROPE_NEOX || table->rotary_dim != cfg->head_dim)
      return set_err(SPISSA_ERR_SHAPE, "the fused decode step needs a llama or gemma table over the whole head");
    for (size_t b = 0; b < batch; ++b)
      if (caches[b]->len >= table->max_positions)
        return set_err(SPISSA_ERR_SHAPE, "position %zu exceeds the rope table (%zu positions)", caches[b]->len,
                       table->max_positions);
  }
  return SPISSA_OK;
}

extern "C" int spissa_decode_step_device(spissa_session *s, const spissa_rope_table *table, const float *d_q,
                                         const float *d_k, const float *d_v, spissa_kv_cache *const *caches,
                                         size_t batch, const spissa_kv_attention_config *cfg, float *d_out) {
  GUARD_BEGIN
  ST_TRY(validate_decode_step(s, table, caches, batch, cfg));
  if (batch == 0) return SPISSA_OK;
  HIP_TRY(hipSetDevice(s->device));
  ST_TRY(run_decode(s, d_q, d_k, d_v, caches, batch, cfg, d_out, table, true));
  for (size_t b = 0; b < batch; ++b) caches[b]->len += 1;
  return SPISSA_OK;
  GUARD_END
}

extern "C" int spissa_gemma_decode_step_device(spissa_session *s, const spissa_rope_table *table,
                                               const float *d_q, const float *d_k, const float *d_v,
                                               spissa_kv_cache *const *caches, size_t batch,
                                               const spissa_kv_attention_config *cfg, const float *d_q_norm,
                                               const float *d_k_norm, float eps, float q_prescale, float *d_out) {
  GUARD_BEGIN
  if (!table || !d_q_norm || !d_k_norm) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  if (table->kind != SPISSA_ROPE_GEMMA)
    return set_err(SPISSA_ERR_ARGUMENT, "the gemma decode step needs a gemma rope table");
  ST_TRY(validate_decode_step(s, table, caches, batch, cfg));
  if (batch == 0) return SPISSA_OK;
  HIP_TRY(hipSetDevice(s->device));
  const GemmaQkNorm norm{d_q_norm, d_k_norm, eps, q_prescale};
  ST_TRY(run_decode(s, d_q, d_k, d_v, caches, batch, cfg, d_out, table, true, nullptr, 0, &norm));
  for (size_t b = 0; b < batch; ++b) caches[b]->len += 1;
  return SPISSA_OK;
  GUARD_END
}

extern "C" int spissa_decode_step_device_noalloc(spissa_session *s, const spissa_rope_table *table,
                                                 const float *d_q, const float *d_k, const float *d_v,
                                                 spissa_kv_cache *const *caches, size_t batch,
                                                 const spissa_kv_attention_config *cfg, float *d_out) {
  GUARD_BEGIN
  ST_TRY(validate_decode_step(s, table, caches, batch, cfg));
  if (!s->scratch) return set_err(SPISSA_ERR_DEVICE, "the session has no scratch array");
  // One split per (sequence, KV head, head block) must fit; run_decode
  // coarsens the splits to the array otherwise.
  const size_t B = std::min<size_t>(batch, kMaxDecodeBatch);
  const size_t single = B * cfg->num_heads * (cfg->head_dim + 2) * sizeof(float);
  if (single > kScratchBytes)
    return set_err(SPISSA_ERR_SHAPE,
                   "decode partials of %zu sequences x %zu heads x head_dim %zu need %zu bytes; the scratch array "
                   "holds %zu",
                   B, cfg->num_heads, cfg->head_dim, single, kScratchBytes);
  if (batch == 0) return SPISSA_OK;
  HIP_TRY(hipSetDevice(s->device));
  ST_TRY(run_decode(s, d_q, d_k, d_v, caches, batch, cfg, d_out, table, true, s->scratch, kScratchBytes));
  for (size_t b = 0; b < batch; ++b) caches[b]->len += 1;
  return SPISSA_OK;
  GUARD_END
}

// The prefill over a chunk whose rows are already the cache's rows
// [P, P + S): every key comes from the cache's bf16 shadow, so P8 covers the
// whole padded key range and no staging buffer is used.
static void plan_prefill_from_shadow(spissa_session *s, const spissa_kv_attention_config *cfg, size_t P,
                                     PrefillArgs &a, PrefillPlan &plan) {
  prefill_args_base(a, cfg, (int)P);
  plan_prefill(a, (int)cfg->head_dim, s->cus, &plan);
  a.P8 = (int)((P + cfg->query_len + 63) & ~(size_t)63);
  a.cap_stage = 0;
  plan.P8 = a.P8;
  plan.cap_stage = 0;
  plan.stage_bytes = 0;
}

// Launches the planned prefill (and its split combine) over the cache's
// shadow, with Q from q (f32) or, when set, qb (scaled bf16).
static int launch_prefill_from_shadow(spissa_session *s, PrefillArgs &a, const spissa_kv_cache *cache, const float *q,
                                      const bf16 *qb, float *out, int D) {
  a.q = q;
  a.qb = qb;
  a.out = out;
  a.kb_cache = cache->kb;
  a.vt_cache = cache->vt;
  a.cap_cache = (long)cache->shadow_cap;
  a.err = s->d_err;
  if (a.splits > 1) {
    const size_t rows = (size_t)a.splits * a.S * a.Hq;
    a.part_o = (float *)s->ppart.p;
    a.part_ml = a.part_o + rows * D;
  }
  HIP_TRY(launch_prefill(s->stream, a, D));
  HIP_TRY(launch_prefill_combine(s->stream, a, D));
  return SPISSA_OK;
}

// The fused prefill step (RoPE, append, attention over the shadow), with the
// Gemma QK-norm folded into the append when `norm` is set.
static int run_prefill_step(spissa_session *s, const spissa_rope_table *table, const float *d_q, const float *d_k,
                            const float *d_v, spissa_kv_cache *cache, const spissa_kv_attention_config *cfg,
                            float *d_out, const GemmaQkNorm *norm) {
  ST_TRY(validate_attention(0, 0, 0, cache, cfg, false));
  size_t n, nl;  // rotary.rs:227-251: the append must fit before anything runs
  ST_TRY(kv_validate_append(cache, 0, 0, cfg->query_len, false, &n, &nl));
  if (cache->session->device != s->device)
    return set_err(SPISSA_ERR_ARGUMENT, "cache lives on device %d, session on %d", cache->session->device, s->device);
  const int D = (int)cfg->head_dim;
  if (!prefill_supported(D) || s->prefill_precision != SPISSA_PREFILL_BF16)
    return set_err(SPISSA_ERR_SHAPE, "the fused prefill step runs the bf16 prefill at head_dim 64, 128 or 256, got %d",
                   D);
  const size_t P = cache->len, S = cfg->query_len;
  if (table) {
    if (table->kind == SPISSA_ROPE_NEOX || table->rotary_dim != cfg->head_dim)
      return set_err(SPISSA_ERR_SHAPE, "the fused prefill step needs a llama or gemma table over the whole head");
    if (P + S > table->max_positions)
      return set_err(SPISSA_ERR_SHAPE, "positions up to %zu exceed the rope table (%zu positions)", P + S,
                     table->max_positions);
  }
  if (!d_q || !d_k || !d_v || !d_out) return set_err(SPISSA_ERR_ARGUMENT, "null buffer");
  HIP_TRY(hipSetDevice(s->device));
  PrefillArgs a;
  PrefillPlan plan;
  plan_prefill_from_shadow(s, cfg, P, a, plan);
  ST_TRY(ensure_shadow(cache, s->stream));
  // Head_dim 64/128 without the QK-norm: the attention kernel rotates and
  // scales the f32 q as it loads it (the same bf16 values), so the append
  // pass stages no q (Llama-3.2-3B 4096-token step: the append pass moves 75
  // MB less). The Gemma form and head_dim 256 stage the normed, rotated q in
  // bf16.
  const bool q_in_kernel = !norm && D <= 128;
  bf16 *qb = nullptr;
  if (!q_in_kernel) {
    ST_TRY(ensure_buf(s, s->qstage, S * cfg->num_heads * cfg->head_dim * sizeof(bf16)));
    qb = (bf16 *)s->qstage.p;
  }
  if (plan.ppart_bytes) ST_TRY(ensure_buf(s, s->ppart, plan.ppart_bytes));
  PrefillNorm pn{};
  if (norm) pn = PrefillNorm{norm->q_norm, norm->k_norm, norm->eps, norm->q_prescale};
  HIP_TRY(launch_prefill_append(s->stream, d_q, d_k, d_v, table ? table->cos : nullptr, table ? table->sin : nullptr,
                                P, S, cfg->kv_heads, cfg->num_heads, cfg->head_dim, cache->keys, cache->values,
                                cache->kb, cache->vt, cache->shadow_cap, qb, a.qk_scale_log2, norm ? &pn : nullptr));
  if (q_in_kernel && table) {
    a.q_cos = table->cos;
    a.q_sin = table->sin;
  }
  ST_TRY(launch_prefill_from_shadow(s, a, cache, d_q, qb, d_out, D));
  cache->len = nl;
  return SPISSA_OK;
}

extern "C" int spissa_prefill_step_device(spissa_session *s, const spissa_rope_table *table, const float *d_q,
                                          const float *d_k, const float *d_v, spissa_kv_cache *cache,
                                          const spissa_kv_attention_config *cfg, float *d_out) {
  GUARD_BEGIN
  if (!s || !cfg || !cache) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  if (cfg->query_len == 1) return spissa_decode_step_device(s, table, d_q, d_k, d_v, &cache, 1, cfg, d_out);
  return run_prefill_step(s, table, d_q, d_k, d_v, cache, cfg, d_out, nullptr);
  GUARD_END
}

extern "C" int spissa_gemma_prefill_step_device(spissa_session *s, const spissa_rope_table *table, const float *d_q,
                                                const float *d_k, const float *d_v, spissa_kv_cache *cache,
                                                const spissa_kv_attention_config *cfg, const float *d_q_norm,
                                                const float *d_k_norm, float eps, float q_prescale, float *d_out) {
  GUARD_BEGIN
  if (!s || !cfg || !cache || !table || !d_q_norm || !d_k_norm) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  if (table->kind != SPISSA_ROPE_GEMMA)
    return set_err(SPISSA_ERR_ARGUMENT, "the gemma prefill step needs a gemma rope table");
  if (cfg->query_len == 1)
    return spissa_gemma_decode_step_device(s, table, d_q, d_k, d_v, &cache, 1, cfg, d_q_norm, d_k_norm, eps,
                                           q_prescale, d_out);
  const GemmaQkNorm norm{d_q_norm, d_k_norm, eps, q_prescale};
  return run_prefill_step(s, table, d_q, d_k, d_v, cache, cfg, d_out, &norm);
  GUARD_END
}

extern "C" int spissa_attention_cached_device(spissa_session *s, const float *d_q, spissa_kv_cache *cache,
                                              const spissa_kv_attention_config *cfg, float *d_out) {
  GUARD_BEGIN
  if (!s || !cfg || !cache) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  if (cfg->query_len < 2)
    return set_err(SPISSA_ERR_SHAPE, "append-first attention needs query_len > 1, got %zu", cfg->query_len);
  if (cache->len < cfg->query_len)
    return set_err(SPISSA_ERR_SHAPE, "the cache holds %zu rows, fewer than the chunk's %zu", cache->len,
                   cfg->query_len);
  const size_t P = cache->len - cfg->query_len, S = cfg->query_len;
  // rotary.rs:483-547 on the call as it would be made before the append
  {
    spissa_kv_cache before = *cache;
    before.len = P;
    ST_TRY(validate_attention(0, 0, 0, &before, cfg, false));
  }
  if (cache->session->device != s->device)
    return set_err(SPISSA_ERR_ARGUMENT, "cache lives on device %d, session on %d", cache->session->device, s->device);
  const int D = (int)cfg->head_dim;
  if (!prefill_supported(D) || s->prefill_precision != SPISSA_PREFILL_BF16)
    return set_err(SPISSA_ERR_SHAPE, "append-first attention runs the bf16 prefill at head_dim 64, 128 or 256, got %d",
                   D);
  if (!d_q || !d_out) return set_err(SPISSA_ERR_ARGUMENT, "null buffer");
  HIP_TRY(hipSetDevice(s->device));
  PrefillArgs a;
  PrefillPlan plan;
  plan_prefill_from_shadow(s, cfg, P, a, plan);
  ST_TRY(ensure_shadow(cache, s->stream));
  if (plan.ppart_bytes) ST_TRY(ensure_buf(s, s->ppart, plan.ppart_bytes));
  // The last key tile reads shadow rows up to the next multiple of 64: they
  // must hold finite values (zeros), whatever earlier, longer contents left.
  const size_t pad_end = (P + S + 63) & ~(size_t)63;
  if (pad_end > P + S)
    HIP_TRY(launch_stage_bf16(s->stream, nullptr, nullptr, 0, pad_end - (P + S), cache->num_heads, cache->head_dim,
                              cache->kb, cache->vt, P + S, cache->shadow_cap));
  return launch_prefill_from_shadow(s, a, cache, d_q, nullptr, d_out, D);
  GUARD_END
}

extern "C" int spissa_plan_attention(const spissa_kv_attention_config *cfg, const size_t *past_lens, size_t batch,
                                     int compute_units, int prefill_precision, int noalloc,
                                     spissa_attention_plan *out) {
  GUARD_BEGIN
  if (!cfg || !past_lens || !out) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  if (batch == 0) return set_err(SPISSA_ERR_ARGUMENT, "a plan needs at least one sequence");
  if (batch > 1 && cfg->query_len != 1)
    return set_err(SPISSA_ERR_SHAPE, "several sequences need query_len == 1, got %zu", cfg->query_len);
  ST_TRY(validate_attention(0, 0, 0, nullptr, cfg, false));
  for (size_t b = 0; b < batch; ++b)
    if (past_lens[b] > (size_t)INT32_MAX / 2 - cfg->query_len)
      return set_err(SPISSA_ERR_SHAPE, "attention sizes exceed the device kernels' limits");
  memset(out, 0, sizeof *out);
  const int D = (int)cfg->head_dim, Hq = (int)cfg->num_heads, Hkv = (int)cfg->kv_heads;
  const int cus = compute_units > 0 ? compute_units : 256;
  if (cfg->query_len == 1 && decode_supported(D, Hq / Hkv)) {
    out->path = SPISSA_KERNEL_DECODE;
    const size_t first = std::min<size_t>(batch, kMaxDecodeBatch);
    if (noalloc && first * cfg->num_heads * (cfg->head_dim + 2) * sizeof(float) > kScratchBytes)
      return set_err(SPISSA_ERR_SHAPE, "decode partials exceed the scratch array (%zu bytes)", kScratchBytes);
    for (size_t b0 = 0; b0 < batch; b0 += kMaxDecodeBatch) {
      const int B = (int)std::min<size_t>(kMaxDecodeBatch, batch - b0);
      int past[kMaxDecodeBatch];
      for (int b = 0; b < B; ++b) past[b] = (int)past_lens[b0 + b];
      DecodePlan p;
      if (!plan_decode(D, Hq, Hkv, cfg->window, past, B, noalloc ? kScratchBytes : 0, &p))
        return set_err(SPISSA_ERR_SHAPE, "decode partials exceed the scratch array (%zu bytes)", kScratchBytes);
      if (b0 == 0) {
        out->heads_per_block = p.RB;
        out->head_blocks = p.HB;
        out->keys_per_split = p.kps;
        out->splits = p.max_splits;
        out->token_split = p.tok_split;
        out->workgroups = p.workgroups;
      }
      out->partial_bytes = std::max(out->partial_bytes, p.partial_bytes);
    }
    return SPISSA_OK;
  }
  if (cfg->query_len > 1 && prefill_precision == SPISSA_PREFILL_BF16 && prefill_supported(D)) {
    out->path = SPISSA_KERNEL_PREFILL_BF16;
    PrefillArgs a;
    prefill_args_base(a, cfg, (int)past_lens[0]);
    PrefillPlan p;
    plan_prefill(a, D, cus, &p);
    out->splits = a.splits;
    out->tiles_per_split = a.tps;
    out->tile_keys = prefill_tile_keys(D);
    out->workgroup_queries = prefill_wg_queries(a, D);
    out->heads_per_block = prefill_wg_heads(a, D);
    out->head_blocks = a.R / out->heads_per_block;
    out->block_waves = a.ksp == 2 ? 2 : 1;
    out->xcd_group = a.xcd_group;
    out->max_tiles = p.tiles;
    out->workgroups = p.workgroups;
    out->partial_bytes = p.ppart_bytes;
    out->stage_bytes = p.stage_bytes;
    return SPISSA_OK;
  }
  out->path = SPISSA_KERNEL_GENERIC;
  return SPISSA_OK;
  GUARD_END
}

extern "C" int spissa_scaled_dot_product_attention_with_cache(const float *q, size_t q_len, const float *current_k,
                                                              size_t k_len, const float *current_v, size_t v_len,
                                                              const spissa_kv_cache *cache,
                                                              const spissa_kv_attention_config *cfg, float *out,
                                                              size_t out_len) {
  GUARD_BEGIN
  if (!cfg) return set_err(SPISSA_ERR_ARGUMENT, "config is null");
  ST_TRY(validate_attention(q_len, k_len, v_len, cache, cfg, true));
  if (out_len != q_len) return set_err(SPISSA_ERR_SHAPE, "output holds %zu floats, need %zu", out_len, q_len);
  if (!q || !current_k || !current_v || !out) return set_err(SPISSA_ERR_ARGUMENT, "null buffer");
  spissa_session *s = nullptr;
  ST_TRY(spissa_default_session(&s));
  if (cache && cache->session->device != s->device)
    return set_err(SPISSA_ERR_ARGUMENT, "cache lives on device %d, the calling thread on %d", cache->session->device,
                   s->device);
  if (cache && cache->session != s) HIP_TRY(hipStreamSynchronize(cache->session->stream));
  float *r[4];
  ST_TRY(io_regions(s, {q_len, k_len, v_len, q_len}, r));
  HIP_TRY(hipSetDevice(s->device));
  ST_TRY(h2d(s, r[0], q, q_len * sizeof(float)));
  ST_TRY(h2d(s, r[1], current_k, k_len * sizeof(float)));
  ST_TRY(h2d(s, r[2], current_v, v_len * sizeof(float)));
  ST_TRY(attention_device_impl(s, r[0], r[1], r[2], cache, cfg, r[3]));
  ST_TRY(spissa_session_sync(s));
  ST_TRY(d2h(s, out, r[3], q_len * sizeof(float)));
  return sync_stream(s);
  GUARD_END
}

extern "C" int spissa_scaled_dot_product_attention(const float *q, size_t q_len, const float *k, size_t k_len,
                                                   const float *v, size_t v_len, size_t seq_len, size_t num_heads,
                                                   size_t head_dim, int causal, float *out, size_t out_len) {
  GUARD_BEGIN
  // ops.rs:246-255
  const size_t expected = seq_len * num_heads * head_dim;
  if (q_len != expected || k_len != expected || v_len != expected)
    return set_err(SPISSA_ERR_SHAPE, "attention shape mismatch: expected %zu, got q=%zu, k=%zu, v=%zu", expected,
                   q_len, k_len, v_len);
  if (out_len != expected) return set_err(SPISSA_ERR_SHAPE, "output holds %zu floats, need %zu", out_len, expected);
  if (expected == 0) return SPISSA_OK;
  spissa_kv_attention_config c = {seq_len, num_heads, num_heads, head_dim, causal, 0};
  return spissa_scaled_dot_product_attention_with_cache(q, q_len, k, k_len, v, v_len, nullptr, &c, out, out_len);
  GUARD_END
}

// ------------------------------------------------------------------------
// Linear projections (streaming/linear.rs:269-576)
// ------------------------------------------------------------------------
struct spissa_linear_weight {
  spissa_session *session = nullptr;
  int dtype = SPISSA_DTYPE_BF16;
  size_t out_features = 0, in_features = 0;
  void *data = nullptr;  // [out, in] row-major in HBM
};

static size_t dtype_size(int dtype) {
  switch (dtype) {
    case SPISSA_DTYPE_F32: return 4;
    case SPISSA_DTYPE_F16: return 2;
    case SPISSA_DTYPE_BF16: return 2;
    default: return 0;
  }
}

extern "C" int spissa_linear_weight_new(spissa_session *s, int dtype, size_t out_features, size_t in_features,
                                        const void *data, size_t data_bytes, spissa_linear_weight **out) {
  GUARD_BEGIN
  if (!s || !out) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  *out = nullptr;
  const size_t es = dtype_size(dtype);
  if (es == 0) return set_err(SPISSA_ERR_INVALID_TENSOR_DATA, "weight dtype %d has no device kernel", dtype);
  size_t elems;
  if (mul_ovf(out_features, in_features, &elems) || elems > (size_t)INT32_MAX * 8)
    return set_err(SPISSA_ERR_SHAPE, "weight element count overflow");
  if (out_features == 0 || in_features == 0 || out_features > INT32_MAX || in_features > INT32_MAX)
    return set_err(SPISSA_ERR_SHAPE, "weight shape [%zu, %zu] is empty or too large", out_features, in_features);
  // streaming/validation.rs:280-287: stored bytes must match shape x dtype
  if (data_bytes != elems * es)
    return set_err(SPISSA_ERR_INVALID_TENSOR_DATA, "weight holds %zu bytes, shape [%zu, %zu] needs %zu", data_bytes,
                   out_features, in_features, elems * es);
  if (!data) return set_err(SPISSA_ERR_ARGUMENT, "data is null");
  std::unique_ptr<spissa_linear_weight> w(new spissa_linear_weight);
  w->session = s;
  w->dtype = dtype;
  w->out_features = out_features;
  w->in_features = in_features;
  HIP_TRY(hipSetDevice(s->device));
  HIP_TRY(hipMalloc(&w->data, data_bytes));
  // host or device source: the runtime resolves the direction from the pointer
  hipError_t e = hipMemcpyAsync(w->data, data, data_bytes, hipMemcpyDefault, s->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
  if (e != hipSuccess) {
    (void)hipFree(w->data);
    return set_err(SPISSA_ERR_DEVICE, "weight upload failed: %s", hipGetErrorString(e));
  }
  *out = w.release();
  session_retain(s);
  return SPISSA_OK;
  GUARD_END
}

extern "C" void spissa_linear_weight_free(spissa_linear_weight *w) {
  if (!w) return;
  spissa_session *s = w->session;
  (void)hipSetDevice(s->device);
  (void)hipStreamSynchronize(s->stream);
  if (w->data) (void)hipFree(w->data);
  delete w;
  session_release(s);
}

static int linear_launch(spissa_session *s, const spissa_linear_weight *w, const float *d_x, const float *d_bias,
                         size_t batch, float *d_out) {
  if (batch == 0) return SPISSA_OK;
  if (batch > INT32_MAX) return set_err(SPISSA_ERR_SHAPE, "batch %zu too large", batch);
  LinearArgs a{};
  a.w = w->data;
  a.x = d_x;
  a.bias = d_bias;
  a.out = d_out;
  a.M = (int)batch;
  a.N = (int)w->out_features;
  a.K = (int)w->in_features;
  a.dtype = w->dtype;
  a.cus = s->cus;
  int path = linear_path(a.dtype, a.M, a.K);
  // the vector kernels read 16-byte pieces of x and of the weight rows
  if (path != kLinearGeneric && (reinterpret_cast<uintptr_t>(d_x) & 15)) path = kLinearGeneric;
  HIP_TRY(hipSetDevice(s->device));
  HIP_TRY(launch_linear(s->stream, a, path));
  return SPISSA_OK;
}

// Several weights applied to the same input (the q, k and v projections):
// one GEMV launch when all take the GEMV on an aligned input, else one
// launch each. Results equal those of separate linear_launch calls.
// norm_w (optional; every weight must take the GEMV): the input RMSNorm
// folded into the projections.
static int linear_launch_multi(spissa_session *s, const spissa_linear_weight *const *w, const float *d_x,
                               size_t batch, float *const *d_out, int n, const float *norm_w = nullptr,
                               float norm_eps = 0.0f) {
  if (batch == 0) return SPISSA_OK;
  if (batch > INT32_MAX) return set_err(SPISSA_ERR_SHAPE, "batch %zu too large", batch);
  if (reinterpret_cast<uintptr_t>(d_x) & 15) {
    if (norm_w) return set_err(SPISSA_ERR_ARGUMENT, "the folded input norm needs a 16-byte aligned input");
    for (int i = 0; i < n; ++i) ST_TRY(linear_launch(s, w[i], d_x, nullptr, batch, d_out[i]));
    return SPISSA_OK;
  }
  LinearArgs a[kMaxLinearSegments];
  for (int i = 0; i < n; ++i) {
    a[i] = LinearArgs{};
    a[i].w = w[i]->data;
    a[i].x = d_x;
    a[i].bias = nullptr;
    a[i].out = d_out[i];
    a[i].M = (int)batch;
    a[i].N = (int)w[i]->out_features;
    a[i].K = (int)w[i]->in_features;
    a[i].dtype = w[i]->dtype;
    a[i].norm_w = norm_w;
    a[i].norm_eps = norm_eps;
    a[i].cus = s->cus;
  }
  HIP_TRY(hipSetDevice(s->device));
  HIP_TRY(launch_linear_multi(s->stream, a, n));
  return SPISSA_OK;
}

extern "C" int spissa_linear(const spissa_linear_weight *w, const float *input, size_t input_len, const float *bias,
                             size_t bias_len, const spissa_linear_config *cfg, float *out, size_t out_len) {
  GUARD_BEGIN
  if (!w || !cfg) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  // streaming/validation.rs:225-247 validate_linear_shapes
  size_t want_in, want_out;
  if (mul_ovf(cfg->batch, cfg->in_features, &want_in) || mul_ovf(cfg->batch, cfg->out_features, &want_out))
    return set_err(SPISSA_ERR_SHAPE, "linear shape overflow");
  if (input_len != want_in)
    return set_err(SPISSA_ERR_SHAPE, "input len %zu does not match batch*in_features = %zu", input_len, want_in);
  if (bias && bias_len != cfg->out_features)
    return set_err(SPISSA_ERR_SHAPE, "bias len %zu does not match out_features %zu", bias_len, cfg->out_features);
  // streaming/validation.rs:258-279 validate_weight_tensor (shape)
  if (w->out_features != cfg->out_features || w->in_features != cfg->in_features)
    return set_err(SPISSA_ERR_SHAPE, "weight shape [%zu, %zu] does not match requested [%zu, %zu]", w->out_features,
                   w->in_features, cfg->out_features, cfg->in_features);
  if (out_len != want_out)
    return set_err(SPISSA_ERR_SHAPE, "output holds %zu floats, need %zu", out_len, want_out);
  if (want_out == 0) return SPISSA_OK;
  if ((want_in && !input) || !out) return set_err(SPISSA_ERR_ARGUMENT, "null buffer");
  spissa_session *s = w->session;
  float *r[3];
  ST_TRY(io_regions(s, {want_in, bias ? cfg->out_features : 0, want_out}, r));
  HIP_TRY(hipSetDevice(s->device));
  ST_TRY(h2d(s, r[0], input, want_in * sizeof(float)));
  if (bias) ST_TRY(h2d(s, r[1], bias, cfg->out_features * sizeof(float)));
  ST_TRY(linear_launch(s, w, r[0], bias ? r[1] : nullptr, cfg->batch, r[2]));
  ST_TRY(d2h(s, out, r[2], want_out * sizeof(float)));
  return sync_stream(s);
  GUARD_END
}

extern "C" int spissa_linear_device(spissa_session *s, const spissa_linear_weight *w, const float *d_input,
                                    const float *d_bias, size_t batch, float *d_out) {
  GUARD_BEGIN
  if (!s || !w) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  if (w->session->device != s->device)
    return set_err(SPISSA_ERR_ARGUMENT, "weight lives on device %d, session on %d", w->session->device, s->device);
  if (batch && (!d_input || !d_out)) return set_err(SPISSA_ERR_ARGUMENT, "null buffer");
  return linear_launch(s, w, d_input, d_bias, batch, d_out);
  GUARD_END
}

// ------------------------------------------------------------------------
// LM head and greedy sampling (streaming/mod.rs:186-287, ops.rs:309-348)
// ------------------------------------------------------------------------
static int argmax_launch(spissa_session *s, const float *d_x, size_t n, int64_t excluded, int *d_token) {
  if (n == 0) return set_err(SPISSA_ERR_INVALID_TENSOR_DATA, "cannot sample from empty logits");
  if (n > (size_t)INT32_MAX - 1024) return set_err(SPISSA_ERR_SHAPE, "%zu logits exceed the device index range", n);
  // ops.rs:326-332: no exclusion, an out-of-range one, or a single logit is
  // plain sample_argmax
  const int excl = (excluded < 0 || (uint64_t)excluded >= n || n <= 1) ? -1 : (int)excluded;
  ST_TRY(ensure_buf(s, s->amax, kArgmaxMaxParts * sizeof(ArgmaxPart)));
  HIP_TRY(hipSetDevice(s->device));
  HIP_TRY(launch_argmax(s->stream, d_x, (int)n, excl, (ArgmaxPart *)s->amax.p, d_token));
  return SPISSA_OK;
}

static int check_lm_table(const spissa_linear_weight *t) {
  if (!t) return set_err(SPISSA_ERR_ARGUMENT, "table is null");
  if (t->dtype != SPISSA_DTYPE_F32 && t->dtype != SPISSA_DTYPE_BF16)
    return set_err(SPISSA_ERR_INVALID_TENSOR_DATA, "LM head table must be f32 or bf16 (dtype %d)", t->dtype);
  return SPISSA_OK;
}

extern "C" int spissa_lm_head_logits(const spissa_linear_weight *table, const float *last_hidden,
                                     size_t last_hidden_len, float *logits, size_t logits_len) {
  GUARD_BEGIN
  ST_TRY(check_lm_table(table));
  if (last_hidden_len != table->in_features)
    return set_err(SPISSA_ERR_SHAPE, "last_hidden holds %zu floats, hidden is %zu", last_hidden_len,
                   table->in_features);
  if (logits_len != table->out_features)
    return set_err(SPISSA_ERR_SHAPE, "logits hold %zu floats, vocab_size is %zu", logits_len, table->out_features);
  if (!last_hidden || !logits) return set_err(SPISSA_ERR_ARGUMENT, "null buffer");
  spissa_session *s = table->session;
  float *r[2];
  ST_TRY(io_regions(s, {last_hidden_len, logits_len}, r));
  HIP_TRY(hipSetDevice(s->device));
  ST_TRY(h2d(s, r[0], last_hidden, last_hidden_len * sizeof(float)));
  ST_TRY(linear_launch(s, table, r[0], nullptr, 1, r[1]));
  ST_TRY(d2h(s, logits, r[1], logits_len * sizeof(float)));
  return sync_stream(s);
  GUARD_END
}

extern "C" int spissa_sample_argmax(spissa_session *s, const float *logits, size_t n, int64_t excluded,
                                    size_t *token) {
  GUARD_BEGIN
  if (!s || !token) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  if (n == 0) return set_err(SPISSA_ERR_INVALID_TENSOR_DATA, "cannot sample from empty logits");
  if (!logits) return set_err(SPISSA_ERR_ARGUMENT, "logits are null");
  float *r[2];
  ST_TRY(io_regions(s, {n, 1}, r));
  HIP_TRY(hipSetDevice(s->device));
  ST_TRY(h2d(s, r[0], logits, n * sizeof(float)));
  ST_TRY(argmax_launch(s, r[0], n, excluded, reinterpret_cast<int *>(r[1])));
  int t = -1;
  ST_TRY(d2h(s, &t, r[1], sizeof(int)));
  ST_TRY(sync_stream(s));
  *token = (size_t)t;
  return SPISSA_OK;
  GUARD_END
}

extern "C" int spissa_argmax_device(spissa_session *s, const float *d_logits, size_t n, int64_t excluded,
                                    int32_t *d_token) {
  GUARD_BEGIN
  if (!s) return set_err(SPISSA_ERR_ARGUMENT, "session is null");
  if (n && (!d_logits || !d_token)) return set_err(SPISSA_ERR_ARGUMENT, "null buffer");
  return argmax_launch(s, d_logits, n, excluded, d_token);
  GUARD_END
}

extern "C" int spissa_lm_head_device(spissa_session *s, const spissa_linear_weight *table, const float *d_hidden,
                                     int64_t excluded, float *d_logits, int32_t *d_token) {
  GUARD_BEGIN
  if (!s) return set_err(SPISSA_ERR_ARGUMENT, "session is null");
  ST_TRY(check_lm_table(table));
  if (table->session->device != s->device)
    return set_err(SPISSA_ERR_ARGUMENT, "table lives on device %d, session on %d", table->session->device, s->device);
  if (!d_hidden || !d_logits) return set_err(SPISSA_ERR_ARGUMENT, "null buffer");
  if (d_token && table->out_features > (size_t)INT32_MAX - 1024)
    return set_err(SPISSA_ERR_SHAPE, "%zu logits exceed the device index range", table->out_features);
  ST_TRY(linear_launch(s, table, d_hidden, nullptr, 1, d_logits));
  if (d_token) ST_TRY(argmax_launch(s, d_logits, table->out_features, excluded, d_token));
  return SPISSA_OK;
  GUARD_END
}

// ------------------------------------------------------------------------
// Attention sublayer (models/gemma/generate.rs:178-312,
// models/llama/generate.rs:200-450)
// ------------------------------------------------------------------------
static int check_weight(const spissa_linear_weight *w, size_t out_f, size_t in_f, const char *name,
                        const spissa_session *s) {
  if (!w) return set_err(SPISSA_ERR_ARGUMENT, "%s weight is null", name);
  if (w->out_features != out_f || w->in_features != in_f)
    return set_err(SPISSA_ERR_SHAPE, "%s weight shape [%zu, %zu] does not match [%zu, %zu]", name, w->out_features,
                   w->in_features, out_f, in_f);
  if (w->session->device != s->device) return set_err(SPISSA_ERR_ARGUMENT, "%s weight lives on another device", name);
  return SPISSA_OK;
}

extern "C" int spissa_attention_sublayer_device(spissa_session *s, const spissa_attention_layer *L, const float *d_x,
                                                size_t S, spissa_kv_cache *cache, float *d_out) {
  GUARD_BEGIN
  if (!s || !L) return set_err(SPISSA_ERR_ARGUMENT, "null argument");
  const size_t H = L->hidden, Hq = L->q_heads, Hkv = L->kv_heads, D = L->head_dim;
  if (!H || !Hq || !Hkv || !D) return set_err(SPISSA_ERR_SHAPE, "sublayer dimensions must be non-zero");
  if (Hq % Hkv != 0) return set_err(SPISSA_ERR_SHAPE, "query heads %zu must be a multiple of kv heads %zu", Hq, Hkv);
  ST_TRY(check_weight(L->q_weight, Hq * D, H, "q", s));
  ST_TRY(check_weight(L->k_weight, Hkv * D, H, "k", s));
  ST_TRY(check_weight(L->v_weight, Hkv * D, H, "v", s));
  ST_TRY(check_weight(L->o_weight, H, Hq * D, "o", s));
  const bool qk_norm = L->d_q_norm != nullptr;
  if (qk_norm != (L->d_k_norm != nullptr)) return set_err(SPISSA_ERR_ARGUMENT, "q and k norms come together");
  if (L->rope && (L->rope->kind == SPISSA_ROPE_NEOX || L->rope->rotary_dim != D || L->rope->device != s->device))
    return set_err(SPISSA_ERR_SHAPE, "the sublayer needs a llama or gemma rope table over the whole head");
  if (qk_norm && (!L->rope || L->rope->kind != SPISSA_ROPE_GEMMA))
    return set_err(SPISSA_ERR_ARGUMENT, "the QK-norm prologue needs a gemma rope table");
  if (!qk_norm && L->q_prescale != 1.0f)
    return set_err(SPISSA_ERR_ARGUMENT, "a q prescale other than 1 comes with the QK-norm prologue");
  const size_t pos = cache ? cache->len : 0;
  if (L->rope && pos + S > L->rope->max_positions)
    return set_err(SPISSA_ERR_SHAPE, "positions %zu..%zu exceed the rope table (%zu positions)", pos, pos + S,
                   L->rope->max_positions);
  if (cache) {
    if (cache->session != s) return set_err(SPISSA_ERR_ARGUMENT, "the cache belongs to another session");
    if (cache->num_heads != Hkv || cache->head_dim != D)
      return set_err(SPISSA_ERR_SHAPE, "cache holds [%zu, %zu] rows, the layer makes [%zu, %zu]", cache->num_heads,
                     cache->head_dim, Hkv, D);
    size_t n, nl;  // rotary.rs:227-251: the append must fit before anything runs
    ST_TRY(kv_validate_append(cache, 0, 0, S, false, &n, &nl));
  }
  if (S == 0) return SPISSA_OK;
  if (!d_x || !d_out) return set_err(SPISSA_ERR_ARGUMENT, "null buffer");
  spissa_kv_attention_config cfg{S, Hq, Hkv, D, L->causal, L->window};
  ST_TRY(validate_attention(0, 0, 0, cache, &cfg, false));

  // workspace: normed x, q, k, v, attention output, o projection
  const size_t sizes[6] = {L->d_input_norm ? S * H : 0, S * Hq * D, S * Hkv * D, S * Hkv * D, S * Hq * D,
                           L->d_post_norm ? S * H : 0};
  size_t total = 0;
  for (size_t n : sizes) total += (n + 63) & ~(size_t)63;
  ST_TRY(ensure_buf(s, s->sub, std::max<size_t>(total, 64) * sizeof(float)));
  float *r[6];
  {
    float *p = (float *)s->sub.p;
    for (int i = 0; i < 6; ++i) {
      r[i] = p;
      p += (sizes[i] + 63) & ~(size_t)63;
    }
  }
  HIP_TRY(hipSetDevice(s->device));
  const float *xn = d_x;
  // At up to four tokens every projection is a GEMV that reads each x row
  // whole: the input RMSNorm folds into it (its launch saved) when the three
  // weights share the GEMV path and the input is 16-byte aligned.
  const float *fold = nullptr;
  if (L->d_input_norm) {
    bool gemv = S <= 4 && (reinterpret_cast<uintptr_t>(d_x) & 15) == 0;
    for (const spissa_linear_weight *w : {L->q_weight, L->k_weight, L->v_weight})
      gemv = gemv && w->dtype == L->q_weight->dtype && linear_path(w->dtype, (long)S, (long)H) == kLinearGemv;
    if (gemv) {
      fold = L->d_input_norm;
    } else {
      HIP_TRY(launch_rms_norm_tree(s->stream, d_x, L->d_input_norm, S, H, L->eps, r[0]));
      xn = r[0];
    }
  }
  float *q = r[1], *k = r[2], *v = r[3], *att = r[4];
  {
    const spissa_linear_weight *const wqkv[3] = {L->q_weight, L->k_weight, L->v_weight};
    float *const oqkv[3] = {q, k, v};
    ST_TRY(linear_launch_multi(s, wqkv, xn, S, oqkv, 3, fold, L->eps));
  }
  if (S == 1 && cache && decode_supported((int)D, (int)(Hq / Hkv)) && decode_cache_fits(cache)) {
    // (QK-norm,) RoPE, attention and append in the fused decode step
    spissa_kv_cache *caches[1] = {cache};
    if (qk_norm)
      ST_TRY(spissa_gemma_decode_step_device(s, L->rope, q, k, v, caches, 1, &cfg, L->d_q_norm, L->d_k_norm, L->eps,
                                             L->q_prescale, att));
    else
      ST_TRY(spissa_decode_step_device(s, L->rope, q, k, v, caches, 1, &cfg, att));
  } else if (S > 1 && cache && prefill_supported((int)D) && s->prefill_precision == SPISSA_PREFILL_BF16) {
    // (QK-norm,) RoPE, append and attention in the fused prefill step
    if (qk_norm)
      ST_TRY(spissa_gemma_prefill_step_device(s, L->rope, q, k, v, cache, &cfg, L->d_q_norm, L->d_k_norm, L->eps,
                                              L->q_prescale, att));
    else
      ST_TRY(spissa_prefill_step_device(s, L->rope, q, k, v, cache, &cfg, att));
  } else {
    if (qk_norm)
      ST_TRY(spissa_gemma_qk_prologue_device(s, L->rope, q, k, S, Hq, Hkv, D, L->d_q_norm, L->d_k_norm, L->eps, pos,
                                             L->q_prescale));
    else if (L->rope)
      ST_TRY(spissa_rope_apply_device(s, L->rope, q, k, S, Hq, Hkv, D, pos));
    ST_TRY(spissa_attention_device(s, q, k, v, cache, &cfg, att));
    if (cache) ST_TRY(spissa_kv_cache_append_device(cache, k, v, S));
  }
  float *proj = L->d_post_norm ? r[5] : d_out;
  ST_TRY(linear_launch(s, L->o_weight, att, nullptr, S, proj));
  if (L->d_post_norm) HIP_TRY(launch_rms_norm_tree(s->stream, proj, L->d_post_norm, S, H, L->eps, d_out));
  return SPISSA_OK;
  GUARD_END
}

