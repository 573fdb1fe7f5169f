// SPDX-License-Identifier: MIT
//! The device-resident KV cache and the attention call over it (feature `hip`).
//!
//! With the `hip` feature, `crate::rotary::KvCache` is this type: the API of
//! the CPU cache (rotary.rs:195-318) one for one, with the rows in HBM through
//! `spissa_hip::DeviceKvCache`, appended in place. The errors keep their
//! variants and messages (the C library reproduces rotary.rs's checks and
//! validates before mutating). `keys()` / `values()` return a host mirror
//! copied from the device on first use after each mutation: the attention
//! call never reads it; tests, rollback checks and debugging do.
//!
//! `attention` is `scaled_dot_product_attention_with_cache` (rotary.rs:335-415)
//! on the MI355X: the split-K f32 decode kernel for query_len == 1, the
//! bf16-MFMA flash prefill for longer chunks at head_dim 64, 128 and 256, and
//! the f32 kernel for other head dims.

use std::fmt;
use std::sync::OnceLock;

use spissa_hip::{AttnConfigC, DeviceKvCache, HipError};

use crate::{Result, RuntimeError};
use crate::rotary::KvAttentionConfig;

/// spissa-hip status -> RuntimeError (crates/spissa-runtime/src/error.rs:6-54).
/// A HIP runtime failure has no variant of its own in the runtime; it is
/// reported as invalid tensor data with the HIP message.
pub(crate) fn runtime_error(e: HipError) -> RuntimeError {
    match e {
        HipError::Shape(m) => RuntimeError::Shape(m),
        HipError::InvalidTensorData(m) => RuntimeError::InvalidTensorData(m),
        HipError::Device(m) | HipError::Argument(m) => RuntimeError::InvalidTensorData(format!("HIP: {m}")),
    }
}

pub struct KvCache {
    device: DeviceKvCache,
    keys: OnceLock<Vec<f32>>,
    values: OnceLock<Vec<f32>>,
}

// The handle is only mutated through `&mut self`; shared references call the
// library's read-only accessors, which are safe from several threads.
unsafe impl Sync for KvCache {}

impl KvCache {
    pub fn new(num_heads: usize, head_dim: usize, max_seq_len: usize) -> Result<Self> {
        let device = DeviceKvCache::new(num_heads, head_dim, max_seq_len).map_err(runtime_error)?;
        Ok(Self { device, keys: OnceLock::new(), values: OnceLock::new() })
    }

    fn invalidate(&mut self) {
        self.keys = OnceLock::new();
        self.values = OnceLock::new();
    }

    pub fn append(&mut self, keys: &[f32], values: &[f32], token_count: usize) -> Result<()> {
        self.device.append(keys, values, token_count).map_err(runtime_error)?;
        self.invalidate();
        Ok(())
    }

    pub fn clear(&mut self) {
        self.device.clear();
        self.invalidate();
    }

    pub fn truncate(&mut self, len: usize) -> Result<()> {
        self.device.truncate(len).map_err(runtime_error)?;
        self.invalidate();
        Ok(())
    }

    pub fn resident_bytes(&self) -> usize {
        self.device.resident_bytes()
    }

    pub fn len(&self) -> usize {
        self.device.len()
    }

    pub fn is_empty(&self) -> bool {
        self.device.is_empty()
    }

    pub fn max_seq_len(&self) -> usize {
        self.device.max_seq_len()
    }

    pub fn num_heads(&self) -> usize {
        self.device.num_heads()
    }

    pub fn head_dim(&self) -> usize {
        self.device.head_dim()
    }

    /// The cached keys `[len, num_heads, head_dim]`, copied from HBM once per
    /// mutation. Panics if the device copy fails (the CPU cache's accessor
    /// cannot fail, so there is no error to return).
    pub fn keys(&self) -> &[f32] {
        self.keys
            .get_or_init(|| self.device.read_keys().unwrap_or_else(|e| panic!("KV cache keys copy failed: {e}")))
    }

    pub fn values(&self) -> &[f32] {
        self.values
            .get_or_init(|| self.device.read_values().unwrap_or_else(|e| panic!("KV cache values copy failed: {e}")))
    }

    /// The device handle, for the fused device-tier calls of spissa-hip.
    pub fn device(&self) -> &DeviceKvCache {
        &self.device
    }

    pub fn device_mut(&mut self) -> &mut DeviceKvCache {
        self.invalidate();
        &mut self.device
    }
}

impl Clone for KvCache {
    fn clone(&self) -> Self {
        Self { device: self.device.clone(), keys: OnceLock::new(), values: OnceLock::new() }
    }
}

impl fmt::Debug for KvCache {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        f.debug_struct("KvCache")
            .field("num_heads", &self.num_heads())
            .field("head_dim", &self.head_dim())
            .field("max_seq_len", &self.max_seq_len())
            .field("len", &self.len())
            .field("device", &"HBM")
            .finish()
    }
}

/// scaled_dot_product_attention_with_cache (rotary.rs:335-415) on the device
/// cache: no window (the reference's semantics), a fresh output vector.
pub(crate) fn attention(
    q: &[f32],
    current_k: &[f32],
    current_v: &[f32],
    cache: Option<&KvCache>,
    config: KvAttentionConfig,
) -> Result<Vec<f32>> {
    let cfg = AttnConfigC::new(config.query_len, config.num_heads, config.kv_heads, config.head_dim, config.causal);
    spissa_hip::sdpa_with_cache(q, current_k, current_v, cache.map(KvCache::device), cfg).map_err(runtime_error)
}

#[cfg(test)]
mod tests {
    use super::*;
    use crate::scaled_dot_product_attention;

    fn ramp(n: usize, scale: f32, offset: f32) -> Vec<f32> {
        (0..n).map(|i| ((i * 7 + 3) % 11) as f32 * scale + offset).collect()
    }

    #[test]
    fn append_over_capacity_leaves_the_device_cache_unchanged() {
        let mut cache = KvCache::new(1, 2, 2).unwrap();
        cache.append(&[1.0, 2.0], &[3.0, 4.0], 1).unwrap();
        let err = cache.append(&[5.0, 6.0, 7.0, 8.0], &[1.0, 1.0, 1.0, 1.0], 2).unwrap_err();
        assert!(matches!(err, RuntimeError::Shape(_)));
        assert_eq!(cache.len(), 1);
        assert_eq!(cache.keys(), &[1.0, 2.0]);
        assert_eq!(cache.values(), &[3.0, 4.0]);
    }

    #[test]
    fn truncate_and_resident_bytes_follow_the_cpu_cache() {
        let mut cache = KvCache::new(1, 3, 4).unwrap();
        cache.append(&ramp(6, 1.0, 0.0), &ramp(6, 2.0, 1.0), 2).unwrap();
        assert_eq!(cache.resident_bytes(), 2 * 3 * 2 * 4);
        cache.truncate(1).unwrap();
        assert_eq!(cache.keys(), &ramp(6, 1.0, 0.0)[..3]);
        assert!(matches!(cache.truncate(2).unwrap_err(), RuntimeError::Shape(_)));
        cache.clear();
        assert!(cache.is_empty());
    }

    /// The rollback of models/llama/session/mod.rs:745-771: remember every
    /// layer's length, append, and on error truncate each cache back. The
    /// device caches must hold exactly their old rows afterwards.
    #[test]
    fn session_rollback_restores_every_layer() {
        let (heads, dim) = (2, 4);
        let width = heads * dim;
        let mut caches: Vec<KvCache> = (0..3).map(|_| KvCache::new(heads, dim, 16).unwrap()).collect();
        for (l, cache) in caches.iter_mut().enumerate() {
            cache.append(&ramp(5 * width, 0.5, l as f32), &ramp(5 * width, 0.25, -(l as f32)), 5).unwrap();
        }
        let before: Vec<(Vec<f32>, Vec<f32>)> =
            caches.iter().map(|c| (c.keys().to_vec(), c.values().to_vec())).collect();
        let old_lens: Vec<usize> = caches.iter().map(KvCache::len).collect();
        for cache in caches.iter_mut() {
            cache.append(&ramp(3 * width, 1.5, 2.0), &ramp(3 * width, -1.0, 0.5), 3).unwrap();
        }
        for (cache, len) in caches.iter_mut().zip(old_lens.iter().copied()) {
            let _ = cache.truncate(len);
        }
        for (cache, (k, v)) in caches.iter().zip(before.iter()) {
            assert_eq!(cache.len(), 5);
            assert_eq!(cache.keys(), k.as_slice());
            assert_eq!(cache.values(), v.as_slice());
        }
    }

    /// rotary.rs:827-851 on the device: the cached decode equals the last row
    /// of the full causal attention (f32 decode kernel, relative 1e-4).
    #[test]
    fn cached_decode_matches_full_recompute() {
        let (seq, heads, dim) = (6, 2, 64);
        let width = heads * dim;
        let q = ramp(seq * width, 0.01, -0.05);
        let k = ramp(seq * width, 0.02, -0.1);
        let v = ramp(seq * width, 0.03, 0.2);
        let full = scaled_dot_product_attention(&q, &k, &v, seq, heads, dim, true).unwrap();
        let mut cache = KvCache::new(heads, dim, seq).unwrap();
        cache.append(&k[..(seq - 1) * width], &v[..(seq - 1) * width], seq - 1).unwrap();
        let cfg = KvAttentionConfig { query_len: 1, num_heads: heads, kv_heads: heads, head_dim: dim, causal: true };
        let got = attention(
            &q[(seq - 1) * width..],
            &k[(seq - 1) * width..],
            &v[(seq - 1) * width..],
            Some(&cache),
            cfg,
        )
        .unwrap();
        let want = &full[(seq - 1) * width..];
        let scale = want.iter().fold(0.0f32, |m, x| m.max(x.abs()));
        let err = got.iter().zip(want).fold(0.0f32, |m, (a, b)| m.max((a - b).abs()));
        assert!(err <= 1e-4 * scale, "relative error {}", err / scale);
    }
}
