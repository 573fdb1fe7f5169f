"""Device fast path: sessions and `_device` entry points on HBM-resident buffers.

Buffers are torch tensors on a ROCm device (float32, contiguous); torch only
supplies device memory and streams here. Calls are asynchronous on the
session's stream; `Session.sync()` waits and reports device-side errors
(an invalid softmax denominator raises InvalidTensorDataError, as
rotary.rs:560-564 does).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence

from . import _ffi
from .errors import ArgumentError, check
from .rotary import KvAttentionConfig, KvCache


def _dev(t, name: str) -> int:
    if t is None:
        return 0
    if not getattr(t, "is_cuda", False):
        raise TypeError(f"{name} must be a device tensor")
    import torch

    if t.dtype != torch.float32 or not t.is_contiguous():
        raise TypeError(f"{name} must be a contiguous float32 tensor")
    return t.data_ptr()


def _dev_i32(t, name: str) -> int:
    if t is None:
        return 0
    if not getattr(t, "is_cuda", False):
        raise TypeError(f"{name} must be a device tensor")
    import torch

    if t.dtype != torch.int32 or t.numel() < 1:
        raise TypeError(f"{name} must be an int32 tensor with at least one element")
    return t.data_ptr()


def plan_attention(config: KvAttentionConfig, past_lens: Sequence[int], compute_units: int = 256,
                   precision: int = _ffi.PREFILL_BF16, noalloc: bool = False) -> dict:
    """The launch geometry spissa_plan_attention reports for one attention call
    (no device needed): kernel path, decode head blocks and key splits, prefill
    tiles and key splits, grid and workspace bytes."""
    lib = _ffi.load()
    past = (_ffi.c_size * max(1, len(past_lens)))(*past_lens)
    cfg = config._c()
    plan = _ffi.AttentionPlanC()
    check(lib.spissa_plan_attention(C.byref(cfg), past, len(past_lens), compute_units, precision,
                                    1 if noalloc else 0, C.byref(plan)))
    return {name: getattr(plan, name) for name, _ in _ffi.AttentionPlanC._fields_}


class RopeTable:
    """A resident cos/sin table (spissa_rope_table_new)."""

    def __init__(self, session: "Session", kind: int, rotary_dim: int, base: float,
                 position_divisor: float = 1.0, freq_scale=None, max_positions: int = 8192):
        import numpy as np

        lib = _ffi.load()
        self._lib = lib
        fs = None
        if freq_scale is not None:
            fs = np.ascontiguousarray(np.asarray(freq_scale, dtype=np.float32))
        h = _ffi.c_void_p()
        check(lib.spissa_rope_table_new(
            session.handle, kind, rotary_dim, base, position_divisor,
            None if fs is None else fs.ctypes.data_as(_ffi.c_float_p), 0 if fs is None else fs.size,
            max_positions, C.byref(h)))
        self._h = h
        self.kind = kind
        self.rotary_dim = rotary_dim
        self.max_positions = max_positions

    @property
    def handle(self):
        return self._h

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            self._lib.spissa_rope_table_free(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class AttentionLayer:
    """One layer's attention sublayer (spissa_attention_layer): the four
    projection weights (spissa_amd.linear.LinearWeight on this session's
    device), the norm multipliers as device tensors (None: that norm is
    absent), the layer's rope table (None: no RoPE), and the attention
    parameters. Mirrors the arguments models/gemma/generate.rs:178-312 and
    models/llama/generate.rs:200-450 take from the model build."""

    hidden: int
    q_heads: int
    kv_heads: int
    head_dim: int
    q_weight: object
    k_weight: object
    v_weight: object
    o_weight: object
    input_norm: object = None
    q_norm: object = None
    k_norm: object = None
    post_norm: object = None
    eps: float = 1e-6
    rope: Optional[RopeTable] = None
    q_prescale: float = 1.0
    causal: bool = True
    window: int = 0

    def _c(self) -> _ffi.AttentionLayerC:
        return _ffi.AttentionLayerC(
            self.hidden, self.q_heads, self.kv_heads, self.head_dim, self.q_weight.handle.value,
            self.k_weight.handle.value, self.v_weight.handle.value, self.o_weight.handle.value,
            _dev(self.input_norm, "input_norm") or None, _dev(self.q_norm, "q_norm") or None,
            _dev(self.k_norm, "k_norm") or None, _dev(self.post_norm, "post_norm") or None, self.eps,
            None if self.rope is None else self.rope.handle.value, self.q_prescale, 1 if self.causal else 0,
            self.window)


class Session:
    """One device, one HIP stream (own or borrowed), one workspace."""

    def __init__(self, device: int = 0, stream=None):
        lib = _ffi.load()
        self._lib = lib
        handle = None
        if stream is not None:
            handle = stream if isinstance(stream, int) else stream.cuda_stream
        h = _ffi.c_void_p()
        check(lib.spissa_session_create(device, handle, C.byref(h)))
        self._h = h
        self.device = device

    @property
    def handle(self):
        if self._h is None or not self._h.value:
            raise ArgumentError("session has been closed")
        return self._h

    @property
    def stream_handle(self) -> int:
        return self._lib.spissa_session_stream(self.handle)

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            self._lib.spissa_session_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sync(self) -> None:
        check(self._lib.spissa_session_sync(self.handle))

    def set_prefill_precision(self, precision: int) -> None:
        check(self._lib.spissa_session_set_prefill_precision(self.handle, precision))

    def kv_cache(self, num_heads: int, head_dim: int, max_seq_len: int) -> KvCache:
        return KvCache(num_heads, head_dim, max_seq_len, session=self)

    def rope_table(self, kind: int, rotary_dim: int, base: float, position_divisor: float = 1.0,
                   freq_scale=None, max_positions: int = 8192) -> RopeTable:
        return RopeTable(self, kind, rotary_dim, base, position_divisor, freq_scale, max_positions)

    def rope_apply(self, table: RopeTable, q, k, seq_len: int, q_heads: int, k_heads: int,
                   head_dim: int, position_offset: int) -> None:
        check(self._lib.spissa_rope_apply_device(self.handle, table.handle, _dev(q, "q"),
                                                 _dev(k, "k"), seq_len, q_heads, k_heads, head_dim,
                                                 position_offset))

    def rms_norm(self, x, weight, rows: int, cols: int, eps: float, out) -> None:
        check(self._lib.spissa_rms_norm_device(self.handle, _dev(x, "x"), _dev(weight, "weight"),
                                               rows, cols, eps, _dev(out, "out")))

    def gemma_qk_prologue(self, table: RopeTable, q, k, seq_len: int, q_heads: int, kv_heads: int,
                          head_dim: int, q_norm, k_norm, eps: float, position_offset: int,
                          q_prescale: float) -> None:
        check(self._lib.spissa_gemma_qk_prologue_device(
            self.handle, table.handle, _dev(q, "q"), _dev(k, "k"), seq_len, q_heads, kv_heads,
            head_dim, _dev(q_norm, "q_norm"), _dev(k_norm, "k_norm"), eps, position_offset,
            q_prescale))

    def attention(self, q, k, v, cache: Optional[KvCache], config: KvAttentionConfig, out) -> None:
        cfg = config._c()
        check(self._lib.spissa_attention_device(
            self.handle, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"),
            None if cache is None else cache.handle, C.byref(cfg), _dev(out, "out")))

    def attention_decode_batch(self, q, k, v, caches: Sequence[Optional[KvCache]],
                               config: KvAttentionConfig, out) -> None:
        arr = (_ffi.c_void_p * max(1, len(caches)))()
        for i, c in enumerate(caches):
            arr[i] = None if c is None else c.handle.value
        cfg = config._c()
        check(self._lib.spissa_attention_decode_batch_device(
            self.handle, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), arr, len(caches), C.byref(cfg),
            _dev(out, "out")))

    def decode_step(self, table: Optional[RopeTable], q, k, v, caches: Sequence[KvCache],
                    config: KvAttentionConfig, out) -> None:
        """Fused RoPE + single-token attention + append for `len(caches)` sequences.

        q [B, Hq, D], k/v [B, Hkv, D] are read-only; every cache gains one token
        holding the rotated key and the value."""
        arr = (_ffi.c_void_p * max(1, len(caches)))()
        for i, c in enumerate(caches):
            arr[i] = c.handle.value
        cfg = config._c()
        check(self._lib.spissa_decode_step_device(
            self.handle, None if table is None else table.handle, _dev(q, "q"), _dev(k, "k"),
            _dev(v, "v"), arr, len(caches), C.byref(cfg), _dev(out, "out")))

    def gemma_decode_step(self, table: RopeTable, q, k, v, caches: Sequence[KvCache], config: KvAttentionConfig,
                          q_norm, k_norm, eps: float, q_prescale: float, out) -> None:
        """The Gemma 3 decode step (spissa_gemma_decode_step_device): QK-norm with the
        [D] weights q_norm / k_norm, Gemma RoPE from `table`, q *= q_prescale, then
        attention and append, in the decode step's two launches; q/k/v read-only."""
        arr = (_ffi.c_void_p * max(1, len(caches)))()
        for i, c in enumerate(caches):
            arr[i] = c.handle.value
        cfg = config._c()
        check(self._lib.spissa_gemma_decode_step_device(
            self.handle, table.handle, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), arr, len(caches), C.byref(cfg),
            _dev(q_norm, "q_norm"), _dev(k_norm, "k_norm"), float(eps), float(q_prescale), _dev(out, "out")))

    def decode_step_noalloc(self, table: Optional[RopeTable], q, k, v, caches: Sequence[KvCache],
                            config: KvAttentionConfig, out) -> None:
        """decode_step through spissa_decode_step_device_noalloc: no device allocation; the
        partials live in the library's static per-GPU scratch array."""
        arr = (_ffi.c_void_p * max(1, len(caches)))()
        for i, c in enumerate(caches):
            arr[i] = c.handle.value
        cfg = config._c()
        check(self._lib.spissa_decode_step_device_noalloc(
            self.handle, None if table is None else table.handle, _dev(q, "q"), _dev(k, "k"),
            _dev(v, "v"), arr, len(caches), C.byref(cfg), _dev(out, "out")))

    def prefill_step(self, table: Optional[RopeTable], q, k, v, cache: KvCache, config: KvAttentionConfig,
                     out) -> None:
        """Fused RoPE + attention + append of a chunk of config.query_len tokens
        (spissa_prefill_step_device): q [S, Hq, D], k/v [S, Hkv, D] read-only;
        the cache gains S rows holding the rotated keys and the values."""
        cfg = config._c()
        check(self._lib.spissa_prefill_step_device(
            self.handle, None if table is None else table.handle, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"),
            cache.handle, C.byref(cfg), _dev(out, "out")))

    def gemma_prefill_step(self, table: RopeTable, q, k, v, cache: KvCache, config: KvAttentionConfig, q_norm,
                           k_norm, eps: float, q_prescale: float, out) -> None:
        """The Gemma 3 prefill step (spissa_gemma_prefill_step_device): QK-norm, Gemma
        RoPE, q *= q_prescale, attention and append of a chunk; q/k/v read-only."""
        cfg = config._c()
        check(self._lib.spissa_gemma_prefill_step_device(
            self.handle, table.handle, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), cache.handle, C.byref(cfg),
            _dev(q_norm, "q_norm"), _dev(k_norm, "k_norm"), float(eps), float(q_prescale), _dev(out, "out")))

    def attention_cached(self, q, cache: KvCache, config: KvAttentionConfig, out) -> None:
        """Append-first attention (spissa_attention_cached_device): the chunk's
        rows are already the cache's last config.query_len rows."""
        cfg = config._c()
        check(self._lib.spissa_attention_cached_device(self.handle, _dev(q, "q"), cache.handle, C.byref(cfg),
                                                       _dev(out, "out")))

    def hbm_read_probe(self, buf, sink) -> None:
        """Reads every byte of the device tensor `buf` once (the streaming-read
        ceiling kernel); `sink` is a float32 device tensor of one element."""
        if not getattr(buf, "is_cuda", False):
            raise TypeError("buf must be a device tensor")
        check(self._lib.spissa_hbm_read_probe_device(self.handle, buf.data_ptr(),
                                                     buf.numel() * buf.element_size(), _dev(sink, "sink")))

    def mfma_rate_probe(self, rounds: int, sink) -> float:
        """Launches the dense-MFMA ceiling kernel (rounds x 8 MFMAs per wave, eight
        waves per CU); returns the launch's FLOP count. `sink`: one float32 on the device."""
        flop = C.c_double()
        check(self._lib.spissa_mfma_rate_probe_device(self.handle, int(rounds), _dev(sink, "sink"), C.byref(flop)))
        return flop.value

    def append(self, cache: KvCache, k, v, token_count: int) -> None:
        cache.append_device(_dev(k, "k"), _dev(v, "v"), token_count)

    def attention_sublayer(self, layer: AttentionLayer, x, seq_len: int, cache: Optional[KvCache], out) -> None:
        """x [seq_len, hidden] -> out [seq_len, hidden]: norm, projections, QK-norm, RoPE at the
        cache's next positions, attention, append, o projection, post norm."""
        lc = layer._c()
        check(self._lib.spissa_attention_sublayer_device(
            self.handle, C.byref(lc), _dev(x, "x"), seq_len, None if cache is None else cache.handle,
            _dev(out, "out")))

    def linear_weight(self, data, dtype: int, out_features: int, in_features: int):
        """A weight resident on this session's device (see spissa_amd.linear.LinearWeight)."""
        from .linear import LinearWeight

        return LinearWeight(data, dtype, out_features, in_features, session=self)

    def linear(self, weight, x, bias, batch: int, out) -> None:
        """out[batch, out] = x[batch, in] x W^T + bias on device tensors (bias may be None)."""
        check(self._lib.spissa_linear_device(self.handle, weight.handle, _dev(x, "x"),
                                             _dev(bias, "bias") or None, batch, _dev(out, "out")))

    def argmax(self, logits, n: int, token, excluded: Optional[int] = None) -> None:
        """token[0] (int32 device tensor) = sample_argmax(logits[:n]) for excluded None, else
        sample_argmax_excluding(logits[:n], excluded) (ops.rs:309-348)."""
        check(self._lib.spissa_argmax_device(self.handle, _dev(logits, "logits"), n,
                                             -1 if excluded is None else excluded, _dev_i32(token, "token")))

    def lm_head(self, table, hidden, logits, token=None, excluded: Optional[int] = None) -> None:
        """logits [vocab] = table x hidden [hidden] (streaming/mod.rs:186-287), then, with a token
        tensor, its argmax as in argmax()."""
        check(self._lib.spissa_lm_head_device(self.handle, table.handle, _dev(hidden, "hidden"),
                                              -1 if excluded is None else excluded, _dev(logits, "logits"),
                                              _dev_i32(token, "token")))
