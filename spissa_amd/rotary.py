"""Host-side mirror of crates/spissa-runtime/src/rotary.rs over the C ABI.

Same names, argument meaning and error variants as the Rust module; buffers
are 1-D float32 numpy arrays where Rust takes `&[f32]` / `&mut [f32]`. The
work runs on the GPU through libspissa_hip.so (drop-in entry points, which
copy host buffers to the device and back and synchronise).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _ffi
from .errors import ArgumentError, check


def _f32(a: np.ndarray, name: str, writable: bool = False) -> np.ndarray:
    if not isinstance(a, np.ndarray) or a.dtype != np.float32 or not a.flags.c_contiguous:
        raise TypeError(f"{name} must be a C-contiguous float32 numpy array")
    if writable and not a.flags.writeable:
        raise TypeError(f"{name} must be writable")
    return a


def _ptr(a: Optional[np.ndarray]):
    if a is None:
        return None
    return a.ctypes.data_as(_ffi.c_float_p)


@dataclass(frozen=True)
class RotaryEmbeddingConfig:
    """rotary.rs:6-14"""

    seq_len: int
    num_heads: int
    head_dim: int
    rotary_dim: int
    base: float
    position_offset: int

    def _c(self) -> _ffi.RotaryConfigC:
        return _ffi.RotaryConfigC(self.seq_len, self.num_heads, self.head_dim, self.rotary_dim,
                                  self.base, self.position_offset)


@dataclass(frozen=True)
class KvAttentionConfig:
    """rotary.rs:320-327, plus `window` (0 = the reference: no sliding window)."""

    query_len: int
    num_heads: int
    kv_heads: int
    head_dim: int
    causal: bool
    window: int = 0

    def _c(self) -> _ffi.AttnConfigC:
        return _ffi.AttnConfigC(self.query_len, self.num_heads, self.kv_heads, self.head_dim,
                                1 if self.causal else 0, self.window)


def gpt_neox_rotary_dim(head_dim: int, rotary_pct: float) -> int:
    """rotary.rs:17-38"""
    out = _ffi.c_size()
    check(_ffi.load().spissa_gpt_neox_rotary_dim(head_dim, rotary_pct, C.byref(out)))
    return out.value


def apply_gpt_neox_rotary_inplace(q: np.ndarray, k: np.ndarray, config: RotaryEmbeddingConfig) -> None:
    """rotary.rs:45-69"""
    _f32(q, "q", True)
    _f32(k, "k", True)
    cfg = config._c()
    check(_ffi.load().spissa_apply_gpt_neox_rotary_inplace(_ptr(q), q.size, _ptr(k), k.size,
                                                           C.byref(cfg)))


def apply_llama_rotary_inplace(q: np.ndarray, k: np.ndarray, q_heads: int, k_heads: int,
                               config: RotaryEmbeddingConfig,
                               freq_scale: Optional[np.ndarray] = None) -> None:
    """rotary.rs:75-125"""
    _f32(q, "q", True)
    _f32(k, "k", True)
    if freq_scale is not None:
        _f32(freq_scale, "freq_scale")
    cfg = config._c()
    check(_ffi.load().spissa_apply_llama_rotary_inplace(
        _ptr(q), q.size, _ptr(k), k.size, q_heads, k_heads, C.byref(cfg), _ptr(freq_scale),
        0 if freq_scale is None else freq_scale.size))


def apply_gemma_rotary_inplace(q: np.ndarray, k: np.ndarray, q_heads: int, k_heads: int,
                               config: RotaryEmbeddingConfig, position_divisor: float) -> None:
    """rotary.rs:137-186"""
    _f32(q, "q", True)
    _f32(k, "k", True)
    cfg = config._c()
    check(_ffi.load().spissa_apply_gemma_rotary_inplace(_ptr(q), q.size, _ptr(k), k.size, q_heads,
                                                        k_heads, C.byref(cfg), position_divisor))


class KvCache:
    """rotary.rs:195-318: append-only per-layer cache, resident in HBM.

    `session` (a spissa_amd.device.Session) binds the cache to that session's
    device and stream; by default it uses the calling thread's default session.
    """

    def __init__(self, num_heads: int, head_dim: int, max_seq_len: int, session=None,
                 _handle: Optional[int] = None):
        lib = _ffi.load()
        self._lib = lib
        self._session = session
        if _handle is not None:
            self._h = _ffi.c_void_p(_handle)
            return
        h = _ffi.c_void_p()
        if session is None:
            check(lib.spissa_kv_cache_new(num_heads, head_dim, max_seq_len, C.byref(h)))
        else:
            check(lib.spissa_kv_cache_new_in(session.handle, num_heads, head_dim, max_seq_len,
                                             C.byref(h)))
        self._h = h

    # KvCache::new is the constructor; keep the Rust spelling available too.
    @classmethod
    def new(cls, num_heads: int, head_dim: int, max_seq_len: int, session=None) -> "KvCache":
        return cls(num_heads, head_dim, max_seq_len, session)

    @property
    def handle(self):
        if self._h is None or not self._h.value:
            raise ArgumentError("KvCache has been closed")
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            self._lib.spissa_kv_cache_free(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def clone(self) -> "KvCache":
        out = _ffi.c_void_p()
        check(self._lib.spissa_kv_cache_clone(self.handle, C.byref(out)))
        return KvCache(0, 0, 0, self._session, _handle=out.value)

    __copy__ = clone

    def append(self, keys: np.ndarray, values: np.ndarray, token_count: int) -> None:
        """rotary.rs:226-256"""
        _f32(keys, "keys")
        _f32(values, "values")
        check(self._lib.spissa_kv_cache_append(self.handle, _ptr(keys), keys.size, _ptr(values),
                                               values.size, token_count))

    def append_device(self, keys_ptr: int, values_ptr: int, token_count: int) -> None:
        """Device-buffer append (asynchronous on the cache's session stream)."""
        check(self._lib.spissa_kv_cache_append_device(self.handle, keys_ptr, values_ptr,
                                                      token_count))

    def clear(self) -> None:
        self._lib.spissa_kv_cache_clear(self.handle)

    def truncate(self, length: int) -> None:
        """rotary.rs:264-278"""
        check(self._lib.spissa_kv_cache_truncate(self.handle, length))

    def resident_bytes(self) -> int:
        return self._lib.spissa_kv_cache_resident_bytes(self.handle)

    def len(self) -> int:
        return self._lib.spissa_kv_cache_len(self.handle)

    def __len__(self) -> int:
        return self.len()

    def is_empty(self) -> bool:
        return bool(self._lib.spissa_kv_cache_is_empty(self.handle))

    def max_seq_len(self) -> int:
        return self._lib.spissa_kv_cache_max_seq_len(self.handle)

    def num_heads(self) -> int:
        return self._lib.spissa_kv_cache_num_heads(self.handle)

    def head_dim(self) -> int:
        return self._lib.spissa_kv_cache_head_dim(self.handle)

    def keys(self) -> np.ndarray:
        """rotary.rs:307-309 (a host copy of the resident rows)."""
        out = np.empty(self.len() * self.num_heads() * self.head_dim(), dtype=np.float32)
        check(self._lib.spissa_kv_cache_read_keys(self.handle, _ptr(out), out.size))
        return out

    def values(self) -> np.ndarray:
        """rotary.rs:311-313"""
        out = np.empty(self.len() * self.num_heads() * self.head_dim(), dtype=np.float32)
        check(self._lib.spissa_kv_cache_read_values(self.handle, _ptr(out), out.size))
        return out

    def device_keys_ptr(self) -> int:
        return self._lib.spissa_kv_cache_device_keys(self.handle)

    def device_values_ptr(self) -> int:
        return self._lib.spissa_kv_cache_device_values(self.handle)


def scaled_dot_product_attention_with_cache(q: np.ndarray, current_k: np.ndarray,
                                            current_v: np.ndarray, cache: Optional[KvCache],
                                            config: KvAttentionConfig) -> np.ndarray:
    """rotary.rs:335-415; returns a fresh [query_len * num_heads * head_dim] array."""
    _f32(q, "q")
    _f32(current_k, "current_k")
    _f32(current_v, "current_v")
    out = np.empty(q.size, dtype=np.float32)
    cfg = config._c()
    check(_ffi.load().spissa_scaled_dot_product_attention_with_cache(
        _ptr(q), q.size, _ptr(current_k), current_k.size, _ptr(current_v), current_v.size,
        None if cache is None else cache.handle, C.byref(cfg), _ptr(out), out.size))
    return out
