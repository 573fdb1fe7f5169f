//! spissa-hip: the MI355X (gfx950) attention path of the Spissa runtime.
//!
//! `sys` declares every function of include/spissa_hip.h one for one (same
//! names, parameter order and C types). The safe layer above it keeps the
//! runtime's argument meaning and error behaviour:
//!
//! - `DeviceKvCache` is `KvCache` (crates/spissa-runtime/src/rotary.rs:195-318)
//!   resident in HBM and appended in place;
//! - `sdpa_with_cache` is `scaled_dot_product_attention_with_cache`
//!   (rotary.rs:335-415) over host q/k/v and a device cache;
//! - `apply_*_rotary_inplace` and `rms_norm` are rotary.rs:17-186 and
//!   ops.rs:159-179, bit-identical to the CPU functions;
//! - `Session` and the `unsafe` device-pointer calls are the fused device
//!   tier (decode and prefill steps, Gemma QK-norm), which a session that
//!   keeps q/k/v on the device calls instead of the three per-layer calls.
//!
//! Status codes map onto `HipError`, which the runtime maps onto
//! `RuntimeError::Shape` / `RuntimeError::InvalidTensorData`
//! (crates/spissa-runtime/src/error.rs:6-54). Nothing here panics across the
//! FFI: every C call returns a status.
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_int, c_void, CStr};
use std::fmt;

/// Raw declarations of include/spissa_hip.h.
pub mod sys {
    use std::ffi::{c_char, c_int, c_long, c_void};

    pub const SPISSA_OK: c_int = 0;
    pub const SPISSA_ERR_SHAPE: c_int = 1;
    pub const SPISSA_ERR_INVALID_TENSOR_DATA: c_int = 2;
    pub const SPISSA_ERR_DEVICE: c_int = 3;
    pub const SPISSA_ERR_ARGUMENT: c_int = 4;

    pub const SPISSA_ROPE_LLAMA: c_int = 0;
    pub const SPISSA_ROPE_GEMMA: c_int = 1;
    pub const SPISSA_ROPE_NEOX: c_int = 2;

    pub const SPISSA_KERNEL_DECODE: c_int = 0;
    pub const SPISSA_KERNEL_PREFILL_BF16: c_int = 1;
    pub const SPISSA_KERNEL_GENERIC: c_int = 2;

    pub const SPISSA_DTYPE_F32: c_int = 0;
    pub const SPISSA_DTYPE_F16: c_int = 1;
    pub const SPISSA_DTYPE_BF16: c_int = 2;

    pub const SPISSA_PREFILL_BF16: c_int = 0;
    pub const SPISSA_PREFILL_F32: c_int = 1;

    #[repr(C)]
    pub struct spissa_session {
        _opaque: [u8; 0],
    }
    #[repr(C)]
    pub struct spissa_kv_cache {
        _opaque: [u8; 0],
    }
    #[repr(C)]
    pub struct spissa_rope_table {
        _opaque: [u8; 0],
    }
    #[repr(C)]
    pub struct spissa_linear_weight {
        _opaque: [u8; 0],
    }

    /// rotary.rs:6-14 RotaryEmbeddingConfig.
    #[repr(C)]
    #[derive(Debug, Clone, Copy, PartialEq)]
    pub struct spissa_rotary_config {
        pub seq_len: usize,
        pub num_heads: usize,
        pub head_dim: usize,
        pub rotary_dim: usize,
        pub base: f32,
        pub position_offset: usize,
    }

    /// rotary.rs:320-327 KvAttentionConfig plus the sliding window (0: none).
    #[repr(C)]
    #[derive(Debug, Clone, Copy, PartialEq, Eq)]
    pub struct spissa_kv_attention_config {
        pub query_len: usize,
        pub num_heads: usize,
        pub kv_heads: usize,
        pub head_dim: usize,
        pub causal: c_int,
        pub window: usize,
    }

    #[repr(C)]
    #[derive(Debug, Clone, Copy, Default, PartialEq, Eq)]
    pub struct spissa_attention_plan {
        pub path: c_int,
        pub heads_per_block: c_int,
        pub head_blocks: c_int,
        pub keys_per_split: c_int,
        pub splits: c_int,
        pub token_split: c_int,
        pub tiles_per_split: c_int,
        pub tile_keys: c_int,
        pub workgroup_queries: c_int,
        pub block_waves: c_int,
        pub xcd_group: c_int,
        pub max_tiles: c_long,
        pub workgroups: usize,
        pub partial_bytes: usize,
        pub stage_bytes: usize,
    }

    /// streaming/mod.rs:511-516 StreamingLinearConfig.
    #[repr(C)]
    #[derive(Debug, Clone, Copy, PartialEq, Eq)]
    pub struct spissa_linear_config {
        pub batch: usize,
        pub in_features: usize,
        pub out_features: usize,
    }

    #[repr(C)]
    #[derive(Debug, Clone, Copy)]
    pub struct spissa_attention_layer {
        pub hidden: usize,
        pub q_heads: usize,
        pub kv_heads: usize,
        pub head_dim: usize,
        pub q_weight: *const spissa_linear_weight,
        pub k_weight: *const spissa_linear_weight,
        pub v_weight: *const spissa_linear_weight,
        pub o_weight: *const spissa_linear_weight,
        pub d_input_norm: *const f32,
        pub d_q_norm: *const f32,
        pub d_k_norm: *const f32,
        pub d_post_norm: *const f32,
        pub eps: f32,
        pub rope: *const spissa_rope_table,
        pub q_prescale: f32,
        pub causal: c_int,
        pub window: usize,
    }

    extern "C" {
        pub fn spissa_last_error() -> *const c_char;
        pub fn spissa_version() -> *const c_char;

        // sessions
        pub fn spissa_session_create(device: c_int, stream: *mut c_void, out: *mut *mut spissa_session) -> c_int;
        pub fn spissa_session_destroy(s: *mut spissa_session);
        pub fn spissa_default_session(out: *mut *mut spissa_session) -> c_int;
        pub fn spissa_session_sync(s: *mut spissa_session) -> c_int;
        pub fn spissa_session_stream(s: *mut spissa_session) -> *mut c_void;
        pub fn spissa_session_device(s: *const spissa_session) -> c_int;
        pub fn spissa_session_set_prefill_precision(s: *mut spissa_session, precision: c_int) -> c_int;

        // KV cache (rotary.rs:195-318)
        pub fn spissa_kv_cache_new(num_heads: usize, head_dim: usize, max_seq_len: usize,
                                   out: *mut *mut spissa_kv_cache) -> c_int;
        pub fn spissa_kv_cache_new_in(s: *mut spissa_session, num_heads: usize, head_dim: usize,
                                      max_seq_len: usize, out: *mut *mut spissa_kv_cache) -> c_int;
        pub fn spissa_kv_cache_free(c: *mut spissa_kv_cache);
        pub fn spissa_kv_cache_clone(c: *const spissa_kv_cache, out: *mut *mut spissa_kv_cache) -> c_int;
        pub fn spissa_kv_cache_append(c: *mut spissa_kv_cache, keys: *const f32, keys_len: usize,
                                      values: *const f32, values_len: usize, token_count: usize) -> c_int;
        pub fn spissa_kv_cache_append_device(c: *mut spissa_kv_cache, d_keys: *const f32,
                                             d_values: *const f32, token_count: usize) -> c_int;
        pub fn spissa_kv_cache_clear(c: *mut spissa_kv_cache);
        pub fn spissa_kv_cache_truncate(c: *mut spissa_kv_cache, len: usize) -> c_int;
        pub fn spissa_kv_cache_len(c: *const spissa_kv_cache) -> usize;
        pub fn spissa_kv_cache_is_empty(c: *const spissa_kv_cache) -> c_int;
        pub fn spissa_kv_cache_max_seq_len(c: *const spissa_kv_cache) -> usize;
        pub fn spissa_kv_cache_num_heads(c: *const spissa_kv_cache) -> usize;
        pub fn spissa_kv_cache_head_dim(c: *const spissa_kv_cache) -> usize;
        pub fn spissa_kv_cache_resident_bytes(c: *const spissa_kv_cache) -> usize;
        pub fn spissa_kv_cache_read_keys(c: *const spissa_kv_cache, dst: *mut f32, dst_len: usize) -> c_int;
        pub fn spissa_kv_cache_read_values(c: *const spissa_kv_cache, dst: *mut f32, dst_len: usize) -> c_int;
        pub fn spissa_kv_cache_device_keys(c: *const spissa_kv_cache) -> *const f32;
        pub fn spissa_kv_cache_device_values(c: *const spissa_kv_cache) -> *const f32;

        // RoPE (rotary.rs:6-193)
        pub fn spissa_gpt_neox_rotary_dim(head_dim: usize, rotary_pct: f32, out: *mut usize) -> c_int;
        pub fn spissa_apply_gpt_neox_rotary_inplace(q: *mut f32, q_len: usize, k: *mut f32, k_len: usize,
                                                    cfg: *const spissa_rotary_config) -> c_int;
        pub fn spissa_apply_llama_rotary_inplace(q: *mut f32, q_len: usize, k: *mut f32, k_len: usize,
                                                 q_heads: usize, k_heads: usize,
                                                 cfg: *const spissa_rotary_config, freq_scale: *const f32,
                                                 freq_scale_len: usize) -> c_int;
        pub fn spissa_apply_gemma_rotary_inplace(q: *mut f32, q_len: usize, k: *mut f32, k_len: usize,
                                                 q_heads: usize, k_heads: usize,
                                                 cfg: *const spissa_rotary_config, position_divisor: f32) -> c_int;
        pub fn spissa_rope_table_new(s: *mut spissa_session, kind: c_int, rotary_dim: usize, base: f32,
                                     position_divisor: f32, freq_scale: *const f32, freq_scale_len: usize,
                                     max_positions: usize, out: *mut *mut spissa_rope_table) -> c_int;
        pub fn spissa_rope_table_free(t: *mut spissa_rope_table);
        pub fn spissa_rope_apply_device(s: *mut spissa_session, t: *const spissa_rope_table, d_q: *mut f32,
                                        d_k: *mut f32, seq_len: usize, q_heads: usize, k_heads: usize,
                                        head_dim: usize, position_offset: usize) -> c_int;

        // RMSNorm and the Gemma QK-norm (ops.rs:159-179, models/gemma)
        pub fn spissa_rms_norm(x: *const f32, x_len: usize, weight: *const f32, weight_len: usize,
                               rows: usize, cols: usize, eps: f32, out: *mut f32, out_len: usize) -> c_int;
        pub fn spissa_rms_norm_device(s: *mut spissa_session, d_x: *const f32, d_weight: *const f32,
                                      rows: usize, cols: usize, eps: f32, d_out: *mut f32) -> c_int;
        pub fn spissa_is_global_layer(layer_idx: usize, sliding_window_pattern: usize) -> c_int;
        pub fn spissa_gemma_qk_prologue_device(s: *mut spissa_session, t: *const spissa_rope_table,
                                               d_q: *mut f32, d_k: *mut f32, seq_len: usize, q_heads: usize,
                                               kv_heads: usize, head_dim: usize, d_q_norm: *const f32,
                                               d_k_norm: *const f32, eps: f32, position_offset: usize,
                                               q_prescale: f32) -> c_int;

        // attention (rotary.rs:335-415, ops.rs:237-291)
        pub fn spissa_scaled_dot_product_attention_with_cache(q: *const f32, q_len: usize,
                                                              current_k: *const f32, k_len: usize,
                                                              current_v: *const f32, v_len: usize,
                                                              cache: *const spissa_kv_cache,
                                                              cfg: *const spissa_kv_attention_config,
                                                              out: *mut f32, out_len: usize) -> c_int;
        pub fn spissa_attention_device(s: *mut spissa_session, d_q: *const f32, d_k: *const f32,
                                       d_v: *const f32, cache: *const spissa_kv_cache,
                                       cfg: *const spissa_kv_attention_config, d_out: *mut f32) -> c_int;
        pub fn spissa_attention_decode_batch_device(s: *mut spissa_session, d_q: *const f32, d_k: *const f32,
                                                    d_v: *const f32, caches: *const *const spissa_kv_cache,
                                                    batch: usize, cfg: *const spissa_kv_attention_config,
                                                    d_out: *mut f32) -> c_int;
        pub fn spissa_decode_step_device(s: *mut spissa_session, table: *const spissa_rope_table,
                                         d_q: *const f32, d_k: *const f32, d_v: *const f32,
                                         caches: *const *mut spissa_kv_cache, batch: usize,
                                         cfg: *const spissa_kv_attention_config, d_out: *mut f32) -> c_int;
        pub fn spissa_gemma_decode_step_device(s: *mut spissa_session, table: *const spissa_rope_table,
                                               d_q: *const f32, d_k: *const f32, d_v: *const f32,
                                               caches: *const *mut spissa_kv_cache, batch: usize,
                                               cfg: *const spissa_kv_attention_config, d_q_norm: *const f32,
                                               d_k_norm: *const f32, eps: f32, q_prescale: f32,
                                               d_out: *mut f32) -> c_int;
        pub fn spissa_decode_step_device_noalloc(s: *mut spissa_session, table: *const spissa_rope_table,
                                                 d_q: *const f32, d_k: *const f32, d_v: *const f32,
                                                 caches: *const *mut spissa_kv_cache, batch: usize,
                                                 cfg: *const spissa_kv_attention_config, d_out: *mut f32) -> c_int;
        pub fn spissa_plan_attention(cfg: *const spissa_kv_attention_config, past_lens: *const usize,
                                     batch: usize, compute_units: c_int, prefill_precision: c_int,
                                     noalloc: c_int, out: *mut spissa_attention_plan) -> c_int;
        pub fn spissa_prefill_step_device(s: *mut spissa_session, table: *const spissa_rope_table,
                                          d_q: *const f32, d_k: *const f32, d_v: *const f32,
                                          cache: *mut spissa_kv_cache, cfg: *const spissa_kv_attention_config,
                                          d_out: *mut f32) -> c_int;
        pub fn spissa_gemma_prefill_step_device(s: *mut spissa_session, table: *const spissa_rope_table,
                                                d_q: *const f32, d_k: *const f32, d_v: *const f32,
                                                cache: *mut spissa_kv_cache,
                                                cfg: *const spissa_kv_attention_config, d_q_norm: *const f32,
                                                d_k_norm: *const f32, eps: f32, q_prescale: f32,
                                                d_out: *mut f32) -> c_int;
        pub fn spissa_attention_cached_device(s: *mut spissa_session, d_q: *const f32, cache: *mut spissa_kv_cache,
                                              cfg: *const spissa_kv_attention_config, d_out: *mut f32) -> c_int;
        pub fn spissa_scaled_dot_product_attention(q: *const f32, q_len: usize, k: *const f32, k_len: usize,
                                                   v: *const f32, v_len: usize, seq_len: usize,
                                                   num_heads: usize, head_dim: usize, causal: c_int,
                                                   out: *mut f32, out_len: usize) -> c_int;

        // projections (streaming/linear.rs:269-576)
        pub fn spissa_linear_weight_new(s: *mut spissa_session, dtype: c_int, out_features: usize,
                                        in_features: usize, data: *const c_void, data_bytes: usize,
                                        out: *mut *mut spissa_linear_weight) -> c_int;
        pub fn spissa_linear_weight_free(w: *mut spissa_linear_weight);
        pub fn spissa_linear(w: *const spissa_linear_weight, input: *const f32, input_len: usize,
                             bias: *const f32, bias_len: usize, cfg: *const spissa_linear_config,
                             out: *mut f32, out_len: usize) -> c_int;
        pub fn spissa_linear_device(s: *mut spissa_session, w: *const spissa_linear_weight,
                                    d_input: *const f32, d_bias: *const f32, batch: usize,
                                    d_out: *mut f32) -> c_int;

        // LM head and greedy sampling (streaming/mod.rs:186-287, ops.rs:309-348)
        pub fn spissa_lm_head_logits(table: *const spissa_linear_weight, last_hidden: *const f32,
                                     last_hidden_len: usize, logits: *mut f32, logits_len: usize) -> c_int;
        pub fn spissa_sample_argmax(s: *mut spissa_session, logits: *const f32, n: usize, excluded: i64,
                                    token: *mut usize) -> c_int;
        pub fn spissa_argmax_device(s: *mut spissa_session, d_logits: *const f32, n: usize, excluded: i64,
                                    d_token: *mut i32) -> c_int;
        pub fn spissa_lm_head_device(s: *mut spissa_session, table: *const spissa_linear_weight,
                                     d_hidden: *const f32, excluded: i64, d_logits: *mut f32,
                                     d_token: *mut i32) -> c_int;

        // the attention sublayer (models/gemma/generate.rs:178-312, models/llama/generate.rs:200-450)
        pub fn spissa_attention_sublayer_device(s: *mut spissa_session, layer: *const spissa_attention_layer,
                                                d_x: *const f32, seq_len: usize, cache: *mut spissa_kv_cache,
                                                d_out: *mut f32) -> c_int;

        // measurement probes (no reference counterpart)
        pub fn spissa_hbm_read_probe_device(s: *mut spissa_session, d_buf: *const c_void, bytes: usize,
                                            d_sink: *mut f32) -> c_int;
        pub fn spissa_mfma_rate_probe_device(s: *mut spissa_session, rounds: c_int, d_sink: *mut f32,
                                             flop: *mut f64) -> c_int;
    }
}

pub use sys::{
    spissa_attention_plan as AttentionPlan, spissa_kv_attention_config as AttnConfigC,
    spissa_linear_config as LinearConfigC, spissa_rotary_config as RotaryConfigC,
};

/// The library's status codes as errors. `Shape` and `InvalidTensorData`
/// carry the reference's messages (rotary.rs, ops.rs); `Device` is a HIP
/// runtime failure and `Argument` a null handle, which the reference cannot
/// produce.
#[derive(Debug, Clone, PartialEq, Eq)]
pub enum HipError {
    Shape(String),
    InvalidTensorData(String),
    Device(String),
    Argument(String),
}

impl fmt::Display for HipError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        match self {
            HipError::Shape(m) => write!(f, "shape mismatch: {m}"),
            HipError::InvalidTensorData(m) => write!(f, "invalid tensor data: {m}"),
            HipError::Device(m) => write!(f, "HIP device error: {m}"),
            HipError::Argument(m) => write!(f, "invalid argument: {m}"),
        }
    }
}

impl std::error::Error for HipError {}

pub type Result<T> = std::result::Result<T, HipError>;

fn last_error() -> String {
    // SAFETY: the library returns a thread-local, NUL-terminated message that
    // stays valid until this thread's next call.
    unsafe {
        let p: *const c_char = sys::spissa_last_error();
        if p.is_null() {
            String::new()
        } else {
            CStr::from_ptr(p).to_string_lossy().into_owned()
        }
    }
}

/// Status code -> Result, with the thread's last message.
pub fn check(code: c_int) -> Result<()> {
    match code {
        sys::SPISSA_OK => Ok(()),
        sys::SPISSA_ERR_SHAPE => Err(HipError::Shape(last_error())),
        sys::SPISSA_ERR_INVALID_TENSOR_DATA => Err(HipError::InvalidTensorData(last_error())),
        sys::SPISSA_ERR_ARGUMENT => Err(HipError::Argument(last_error())),
        _ => Err(HipError::Device(last_error())),
    }
}

/// The library version string.
pub fn version() -> String {
    // SAFETY: a static NUL-terminated string.
    unsafe { CStr::from_ptr(sys::spissa_version()).to_string_lossy().into_owned() }
}

impl AttnConfigC {
    /// rotary.rs:320-327 with no window (the reference's semantics).
    pub fn new(query_len: usize, num_heads: usize, kv_heads: usize, head_dim: usize, causal: bool) -> Self {
        Self { query_len, num_heads, kv_heads, head_dim, causal: causal as c_int, window: 0 }
    }
    /// The sliding-window extension: keys j with i - W < j <= i for a query at i.
    pub fn with_window(mut self, window: usize) -> Self {
        self.window = window;
        self
    }
}

// ---- sessions ----

/// One device and one HIP stream. Device-tier calls are asynchronous on the
/// stream; `sync` waits and reports a device-side softmax error.
pub struct Session {
    raw: *mut sys::spissa_session,
    owned: bool,
}

// The library serialises a session's work on its stream; a session may move
// between threads but not be shared without synchronisation.
unsafe impl Send for Session {}

impl Session {
    /// A session on `device` with a stream of its own.
    pub fn new(device: i32) -> Result<Self> {
        let mut raw = std::ptr::null_mut();
        check(unsafe { sys::spissa_session_create(device, std::ptr::null_mut(), &mut raw) })?;
        Ok(Self { raw, owned: true })
    }
    /// A session on an existing `hipStream_t` (not owned).
    ///
    /// # Safety
    /// `stream` must be a valid stream of `device` for the session's lifetime.
    pub unsafe fn with_stream(device: i32, stream: *mut c_void) -> Result<Self> {
        let mut raw = std::ptr::null_mut();
        check(sys::spissa_session_create(device, stream, &mut raw))?;
        Ok(Self { raw, owned: true })
    }
    /// The calling thread's default session (the one the drop-in calls use).
    pub fn thread_default() -> Result<Self> {
        let mut raw = std::ptr::null_mut();
        check(unsafe { sys::spissa_default_session(&mut raw) })?;
        Ok(Self { raw, owned: false })
    }
    pub fn sync(&self) -> Result<()> {
        check(unsafe { sys::spissa_session_sync(self.raw) })
    }
    pub fn stream(&self) -> *mut c_void {
        unsafe { sys::spissa_session_stream(self.raw) }
    }
    pub fn device(&self) -> i32 {
        unsafe { sys::spissa_session_device(self.raw) }
    }
    pub fn set_prefill_precision(&self, precision: c_int) -> Result<()> {
        check(unsafe { sys::spissa_session_set_prefill_precision(self.raw, precision) })
    }
    pub fn raw(&self) -> *mut sys::spissa_session {
        self.raw
    }
}

impl Drop for Session {
    fn drop(&mut self) {
        if self.owned {
            unsafe { sys::spissa_session_destroy(self.raw) }
        }
    }
}

// ---- the device KV cache (rotary.rs:195-318) ----

/// `KvCache` resident in HBM: `[max_seq_len, num_heads, head_dim]` f32 keys
/// and values, appended in place; the first `len` rows are byte-identical to
/// the CPU cache's `keys()` / `values()`.
pub struct DeviceKvCache(*mut sys::spissa_kv_cache);

unsafe impl Send for DeviceKvCache {}

impl DeviceKvCache {
    /// rotary.rs:206-224 KvCache::new, on the thread's default session.
    pub fn new(num_heads: usize, head_dim: usize, max_seq_len: usize) -> Result<Self> {
        let mut h = std::ptr::null_mut();
        check(unsafe { sys::spissa_kv_cache_new(num_heads, head_dim, max_seq_len, &mut h) })?;
        Ok(Self(h))
    }
    /// The same, bound to `session` (for the device tier).
    pub fn new_in(session: &Session, num_heads: usize, head_dim: usize, max_seq_len: usize) -> Result<Self> {
        let mut h = std::ptr::null_mut();
        check(unsafe { sys::spissa_kv_cache_new_in(session.raw, num_heads, head_dim, max_seq_len, &mut h) })?;
        Ok(Self(h))
    }
    /// rotary.rs:226-256 KvCache::append (validates before mutating).
    pub fn append(&mut self, keys: &[f32], values: &[f32], token_count: usize) -> Result<()> {
        check(unsafe {
            sys::spissa_kv_cache_append(self.0, keys.as_ptr(), keys.len(), values.as_ptr(), values.len(), token_count)
        })
    }
    /// Append from device buffers of `token_count * num_heads * head_dim` floats.
    ///
    /// # Safety
    /// Both pointers must be device memory of at least that many floats.
    pub unsafe fn append_device(&mut self, d_keys: *const f32, d_values: *const f32, token_count: usize) -> Result<()> {
        check(sys::spissa_kv_cache_append_device(self.0, d_keys, d_values, token_count))
    }
    /// rotary.rs:258-262 KvCache::clear.
    pub fn clear(&mut self) {
        unsafe { sys::spissa_kv_cache_clear(self.0) }
    }
    /// rotary.rs:264-278 KvCache::truncate (growing is a Shape error).
    pub fn truncate(&mut self, len: usize) -> Result<()> {
        check(unsafe { sys::spissa_kv_cache_truncate(self.0, len) })
    }
    pub fn len(&self) -> usize {
        unsafe { sys::spissa_kv_cache_len(self.0) }
    }
    pub fn is_empty(&self) -> bool {
        unsafe { sys::spissa_kv_cache_is_empty(self.0) != 0 }
    }
    pub fn max_seq_len(&self) -> usize {
        unsafe { sys::spissa_kv_cache_max_seq_len(self.0) }
    }
    pub fn num_heads(&self) -> usize {
        unsafe { sys::spissa_kv_cache_num_heads(self.0) }
    }
    pub fn head_dim(&self) -> usize {
        unsafe { sys::spissa_kv_cache_head_dim(self.0) }
    }
    /// rotary.rs:280-285: len * num_heads * head_dim * 2 * 4.
    pub fn resident_bytes(&self) -> usize {
        unsafe { sys::spissa_kv_cache_resident_bytes(self.0) }
    }
    /// The first len rows of the keys, copied to the host (backs `keys()`).
    pub fn read_keys(&self) -> Result<Vec<f32>> {
        let mut dst = vec![0.0f32; self.len() * self.num_heads() * self.head_dim()];
        check(unsafe { sys::spissa_kv_cache_read_keys(self.0, dst.as_mut_ptr(), dst.len()) })?;
        Ok(dst)
    }
    /// The first len rows of the values, copied to the host (backs `values()`).
    pub fn read_values(&self) -> Result<Vec<f32>> {
        let mut dst = vec![0.0f32; self.len() * self.num_heads() * self.head_dim()];
        check(unsafe { sys::spissa_kv_cache_read_values(self.0, dst.as_mut_ptr(), dst.len()) })?;
        Ok(dst)
    }
    /// Device base pointers of the resident buffers.
    pub fn device_keys(&self) -> *const f32 {
        unsafe { sys::spissa_kv_cache_device_keys(self.0) }
    }
    pub fn device_values(&self) -> *const f32 {
        unsafe { sys::spissa_kv_cache_device_values(self.0) }
    }
    pub fn raw(&self) -> *const sys::spissa_kv_cache {
        self.0
    }
    pub fn raw_mut(&mut self) -> *mut sys::spissa_kv_cache {
        self.0
    }
    /// #[derive(Clone)] of rotary.rs:195, reporting a failed device copy
    /// (`Clone::clone` panics on it instead).
    pub fn try_clone(&self) -> Result<Self> {
        let mut h = std::ptr::null_mut();
        check(unsafe { sys::spissa_kv_cache_clone(self.0, &mut h) })?;
        Ok(Self(h))
    }
}

impl Clone for DeviceKvCache {
    fn clone(&self) -> Self {
        self.try_clone().unwrap_or_else(|e| panic!("KV cache clone failed: {e}"))
    }
}

impl Drop for DeviceKvCache {
    fn drop(&mut self) {
        unsafe { sys::spissa_kv_cache_free(self.0) }
    }
}

impl fmt::Debug for DeviceKvCache {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        f.debug_struct("DeviceKvCache")
            .field("num_heads", &self.num_heads())
            .field("head_dim", &self.head_dim())
            .field("max_seq_len", &self.max_seq_len())
            .field("len", &self.len())
            .finish()
    }
}

// ---- drop-in host calls ----

/// rotary.rs:335-415 scaled_dot_product_attention_with_cache: host q/k/v,
/// the cache on the device, a fresh output vector.
pub fn sdpa_with_cache(q: &[f32], current_k: &[f32], current_v: &[f32], cache: Option<&DeviceKvCache>,
                       cfg: AttnConfigC) -> Result<Vec<f32>> {
    let n = cfg
        .query_len
        .checked_mul(cfg.num_heads)
        .and_then(|x| x.checked_mul(cfg.head_dim))
        .ok_or_else(|| HipError::Shape("attention output length overflow".to_string()))?;
    let mut out = vec![0.0f32; n];
    check(unsafe {
        sys::spissa_scaled_dot_product_attention_with_cache(
            q.as_ptr(), q.len(), current_k.as_ptr(), current_k.len(), current_v.as_ptr(), current_v.len(),
            cache.map_or(std::ptr::null(), |c| c.raw()), &cfg, out.as_mut_ptr(), out.len())
    })?;
    Ok(out)
}

/// ops.rs:237-291 scaled_dot_product_attention (cacheless MHA).
pub fn scaled_dot_product_attention(q: &[f32], k: &[f32], v: &[f32], seq_len: usize, num_heads: usize,
                                    head_dim: usize, causal: bool) -> Result<Vec<f32>> {
    let mut out = vec![0.0f32; q.len()];
    check(unsafe {
        sys::spissa_scaled_dot_product_attention(q.as_ptr(), q.len(), k.as_ptr(), k.len(), v.as_ptr(), v.len(),
                                                 seq_len, num_heads, head_dim, causal as c_int,
                                                 out.as_mut_ptr(), out.len())
    })?;
    Ok(out)
}

/// rotary.rs:75-125 apply_llama_rotary_inplace (`freq_scale` None: no LongRoPE).
pub fn apply_llama_rotary_inplace(q: &mut [f32], k: &mut [f32], q_heads: usize, k_heads: usize,
                                  cfg: RotaryConfigC, freq_scale: Option<&[f32]>) -> Result<()> {
    let (fp, fl) = freq_scale.map_or((std::ptr::null(), 0), |f| (f.as_ptr(), f.len()));
    check(unsafe {
        sys::spissa_apply_llama_rotary_inplace(q.as_mut_ptr(), q.len(), k.as_mut_ptr(), k.len(), q_heads, k_heads,
                                               &cfg, fp, fl)
    })
}

/// rotary.rs:137-186 apply_gemma_rotary_inplace.
pub fn apply_gemma_rotary_inplace(q: &mut [f32], k: &mut [f32], q_heads: usize, k_heads: usize,
                                  cfg: RotaryConfigC, position_divisor: f32) -> Result<()> {
    check(unsafe {
        sys::spissa_apply_gemma_rotary_inplace(q.as_mut_ptr(), q.len(), k.as_mut_ptr(), k.len(), q_heads, k_heads,
                                               &cfg, position_divisor)
    })
}

/// rotary.rs:45-69 apply_gpt_neox_rotary_inplace.
pub fn apply_gpt_neox_rotary_inplace(q: &mut [f32], k: &mut [f32], cfg: RotaryConfigC) -> Result<()> {
    check(unsafe { sys::spissa_apply_gpt_neox_rotary_inplace(q.as_mut_ptr(), q.len(), k.as_mut_ptr(), k.len(), &cfg) })
}

/// rotary.rs:17-38 gpt_neox_rotary_dim.
pub fn gpt_neox_rotary_dim(head_dim: usize, rotary_pct: f32) -> Result<usize> {
    let mut out = 0usize;
    check(unsafe { sys::spissa_gpt_neox_rotary_dim(head_dim, rotary_pct, &mut out) })?;
    Ok(out)
}

/// ops.rs:159-179 rms_norm (sequential sum of squares per row).
pub fn rms_norm(x: &[f32], weight: &[f32], rows: usize, cols: usize, eps: f32) -> Result<Vec<f32>> {
    let mut out = vec![0.0f32; x.len()];
    check(unsafe {
        sys::spissa_rms_norm(x.as_ptr(), x.len(), weight.as_ptr(), weight.len(), rows, cols, eps, out.as_mut_ptr(),
                             out.len())
    })?;
    Ok(out)
}

/// models/gemma/model.rs:46-51 is_global_layer.
pub fn is_global_layer(layer_idx: usize, sliding_window_pattern: usize) -> bool {
    unsafe { sys::spissa_is_global_layer(layer_idx, sliding_window_pattern) != 0 }
}

/// The launch geometry one attention call will use (host arithmetic only).
pub fn plan_attention(cfg: &AttnConfigC, past_lens: &[usize], noalloc: bool) -> Result<AttentionPlan> {
    let mut plan = AttentionPlan::default();
    check(unsafe {
        sys::spissa_plan_attention(cfg, past_lens.as_ptr(), past_lens.len(), 0, sys::SPISSA_PREFILL_BF16,
                                   noalloc as c_int, &mut plan)
    })?;
    Ok(plan)
}

// ---- the device tier ----

/// A resident cos/sin table (computed on the host with the reference's
/// formulas, so device RoPE is bit-identical to the drop-in call).
pub struct RopeTable(*mut sys::spissa_rope_table);

unsafe impl Send for RopeTable {}

impl RopeTable {
    /// kind: sys::SPISSA_ROPE_{LLAMA,GEMMA,NEOX}; positions [0, max_positions).
    pub fn new(session: &Session, kind: c_int, rotary_dim: usize, base: f32, position_divisor: f32,
               freq_scale: Option<&[f32]>, max_positions: usize) -> Result<Self> {
        let (fp, fl) = freq_scale.map_or((std::ptr::null(), 0), |f| (f.as_ptr(), f.len()));
        let mut h = std::ptr::null_mut();
        check(unsafe {
            sys::spissa_rope_table_new(session.raw, kind, rotary_dim, base, position_divisor, fp, fl, max_positions,
                                       &mut h)
        })?;
        Ok(Self(h))
    }
    pub fn raw(&self) -> *const sys::spissa_rope_table {
        self.0
    }
}

impl Drop for RopeTable {
    fn drop(&mut self) {
        unsafe { sys::spissa_rope_table_free(self.0) }
    }
}

/// Pointers of the caches a batched device call appends to.
fn cache_ptrs(caches: &mut [&mut DeviceKvCache]) -> Vec<*mut sys::spissa_kv_cache> {
    caches.iter_mut().map(|c| c.raw_mut()).collect()
}

/// One fused decode step of one layer for `caches.len()` sequences: RoPE of q
/// and k at each cache's length (table None: none), attention, append of the
/// rotated key and the value (models/llama/generate.rs:373-416 per layer).
///
/// # Safety
/// d_q [B, Hq, d], d_k and d_v [B, Hkv, d], d_out [B, Hq, d] must be device
/// buffers that stay valid until the session's stream has run the call.
pub unsafe fn decode_step(session: &Session, table: Option<&RopeTable>, d_q: *const f32, d_k: *const f32,
                          d_v: *const f32, caches: &mut [&mut DeviceKvCache], cfg: &AttnConfigC,
                          d_out: *mut f32) -> Result<()> {
    let ptrs = cache_ptrs(caches);
    check(sys::spissa_decode_step_device(session.raw, table.map_or(std::ptr::null(), |t| t.raw()), d_q, d_k, d_v,
                                         ptrs.as_ptr(), ptrs.len(), cfg, d_out))
}

/// The Gemma 3 decode step: QK-norm, Gemma RoPE, q prescale, attention,
/// append (models/gemma/generate.rs:232-295), in the same two launches.
///
/// # Safety
/// As `decode_step`; d_q_norm and d_k_norm are device [head_dim] weights.
pub unsafe fn gemma_decode_step(session: &Session, table: &RopeTable, d_q: *const f32, d_k: *const f32,
                                d_v: *const f32, caches: &mut [&mut DeviceKvCache], cfg: &AttnConfigC,
                                d_q_norm: *const f32, d_k_norm: *const f32, eps: f32, q_prescale: f32,
                                d_out: *mut f32) -> Result<()> {
    let ptrs = cache_ptrs(caches);
    check(sys::spissa_gemma_decode_step_device(session.raw, table.raw(), d_q, d_k, d_v, ptrs.as_ptr(), ptrs.len(),
                                               cfg, d_q_norm, d_k_norm, eps, q_prescale, d_out))
}

/// `decode_step` with its partials in the library's static per-GPU array:
/// no device allocation (for graph capture). Calls on one GPU must not overlap.
///
/// # Safety
/// As `decode_step`.
pub unsafe fn decode_step_noalloc(session: &Session, table: Option<&RopeTable>, d_q: *const f32,
                                  d_k: *const f32, d_v: *const f32, caches: &mut [&mut DeviceKvCache],
                                  cfg: &AttnConfigC, d_out: *mut f32) -> Result<()> {
    let ptrs = cache_ptrs(caches);
    check(sys::spissa_decode_step_device_noalloc(session.raw, table.map_or(std::ptr::null(), |t| t.raw()), d_q, d_k,
                                                 d_v, ptrs.as_ptr(), ptrs.len(), cfg, d_out))
}

/// One fused prefill (or chunk) step: RoPE at the cache's length, append of
/// the chunk (f32 rows and the bf16 operands), bf16-MFMA attention.
///
/// # Safety
/// d_q [S, Hq, d], d_k and d_v [S, Hkv, d], d_out [S, Hq, d] device buffers.
pub unsafe fn prefill_step(session: &Session, table: Option<&RopeTable>, d_q: *const f32, d_k: *const f32,
                           d_v: *const f32, cache: &mut DeviceKvCache, cfg: &AttnConfigC,
                           d_out: *mut f32) -> Result<()> {
    check(sys::spissa_prefill_step_device(session.raw, table.map_or(std::ptr::null(), |t| t.raw()), d_q, d_k, d_v,
                                          cache.raw_mut(), cfg, d_out))
}

/// The Gemma 3 prefill (or chunk) step: QK-norm, Gemma RoPE, prescale,
/// append, attention.
///
/// # Safety
/// As `prefill_step`; d_q_norm and d_k_norm are device [head_dim] weights.
pub unsafe fn gemma_prefill_step(session: &Session, table: &RopeTable, d_q: *const f32, d_k: *const f32,
                                 d_v: *const f32, cache: &mut DeviceKvCache, cfg: &AttnConfigC,
                                 d_q_norm: *const f32, d_k_norm: *const f32, eps: f32, q_prescale: f32,
                                 d_out: *mut f32) -> Result<()> {
    check(sys::spissa_gemma_prefill_step_device(session.raw, table.raw(), d_q, d_k, d_v, cache.raw_mut(), cfg,
                                                d_q_norm, d_k_norm, eps, q_prescale, d_out))
}

/// rotary.rs:335-415 on device buffers, asynchronous on the session stream.
///
/// # Safety
/// d_q [S, Hq, d], d_k and d_v [S, Hkv, d], d_out [S, Hq, d] device buffers.
pub unsafe fn attention_device(session: &Session, d_q: *const f32, d_k: *const f32, d_v: *const f32,
                               cache: Option<&DeviceKvCache>, cfg: &AttnConfigC, d_out: *mut f32) -> Result<()> {
    check(sys::spissa_attention_device(session.raw, d_q, d_k, d_v, cache.map_or(std::ptr::null(), |c| c.raw()), cfg,
                                       d_out))
}

// ---- projections, LM head and sampling ----

/// A weight resident in HBM (streaming_tile_linear_from_model's weight,
/// uploaded once), row-major [out_features, in_features].
pub struct DeviceLinearWeight(*mut sys::spissa_linear_weight);

unsafe impl Send for DeviceLinearWeight {}

impl DeviceLinearWeight {
    /// `raw` holds out_features * in_features little-endian elements of dtype
    /// (sys::SPISSA_DTYPE_{F32,F16,BF16}).
    pub fn upload(session: &Session, dtype: c_int, out_features: usize, in_features: usize, raw: &[u8])
                  -> Result<Self> {
        let mut h = std::ptr::null_mut();
        check(unsafe {
            sys::spissa_linear_weight_new(session.raw, dtype, out_features, in_features, raw.as_ptr() as *const c_void,
                                          raw.len(), &mut h)
        })?;
        Ok(Self(h))
    }
    /// streaming/linear.rs:269-576 on host buffers.
    pub fn linear(&self, input: &[f32], bias: Option<&[f32]>, cfg: LinearConfigC) -> Result<Vec<f32>> {
        let n = cfg
            .batch
            .checked_mul(cfg.out_features)
            .ok_or_else(|| HipError::Shape("linear output length overflow".to_string()))?;
        let mut out = vec![0.0f32; n];
        let (bp, bl) = bias.map_or((std::ptr::null(), 0), |b| (b.as_ptr(), b.len()));
        check(unsafe {
            sys::spissa_linear(self.0, input.as_ptr(), input.len(), bp, bl, &cfg, out.as_mut_ptr(), out.len())
        })?;
        Ok(out)
    }
    /// streaming/mod.rs:186-287 lm_head_logits_parallel[_bf16] over this table.
    pub fn lm_head_logits(&self, last_hidden: &[f32], vocab_size: usize) -> Result<Vec<f32>> {
        let mut logits = vec![0.0f32; vocab_size];
        check(unsafe {
            sys::spissa_lm_head_logits(self.0, last_hidden.as_ptr(), last_hidden.len(), logits.as_mut_ptr(),
                                       logits.len())
        })?;
        Ok(logits)
    }
    pub fn raw(&self) -> *const sys::spissa_linear_weight {
        self.0
    }
}

impl Drop for DeviceLinearWeight {
    fn drop(&mut self) {
        unsafe { sys::spissa_linear_weight_free(self.0) }
    }
}

/// ops.rs:309-324 sample_argmax (None) and ops.rs:326-348
/// sample_argmax_excluding (Some), on the thread's default session.
pub fn sample_argmax_excluding(logits: &[f32], excluded: Option<usize>) -> Result<usize> {
    let s = Session::thread_default()?;
    let mut token = 0usize;
    let ex = excluded.map_or(-1i64, |e| i64::try_from(e).unwrap_or(i64::MAX));
    check(unsafe { sys::spissa_sample_argmax(s.raw, logits.as_ptr(), logits.len(), ex, &mut token) })?;
    Ok(token)
}
