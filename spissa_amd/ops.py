"""Host-side mirror of the ops the attention path uses
(crates/spissa-runtime/src/ops.rs:159-179, 237-291;
crates/spissa-runtime/src/models/gemma/model.rs:46-51)."""
from __future__ import annotations

import numpy as np

from . import _ffi
from .errors import check
from .rotary import _f32, _ptr


def rms_norm(x: np.ndarray, weight: np.ndarray, rows: int, cols: int, eps: float) -> np.ndarray:
    """ops.rs:159-179 (bit-identical on the GPU: sequential sum of squares per row)."""
    _f32(x, "x")
    _f32(weight, "weight")
    out = np.empty(x.size, dtype=np.float32)
    check(_ffi.load().spissa_rms_norm(_ptr(x), x.size, _ptr(weight), weight.size, rows, cols, eps,
                                      _ptr(out), out.size))
    return out


def scaled_dot_product_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, seq_len: int,
                                 num_heads: int, head_dim: int, causal: bool) -> np.ndarray:
    """ops.rs:237-291 (cacheless MHA)."""
    for a, n in ((q, "q"), (k, "k"), (v, "v")):
        _f32(a, n)
    out = np.empty(seq_len * num_heads * head_dim, dtype=np.float32)
    check(_ffi.load().spissa_scaled_dot_product_attention(
        _ptr(q), q.size, _ptr(k), k.size, _ptr(v), v.size, seq_len, num_heads, head_dim,
        1 if causal else 0, _ptr(out), out.size))
    return out


def is_global_layer(layer_idx: int, sliding_window_pattern: int) -> bool:
    """models/gemma/model.rs:46-51"""
    return bool(_ffi.load().spissa_is_global_layer(layer_idx, sliding_window_pattern))
