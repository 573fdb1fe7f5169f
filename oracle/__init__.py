"""CPU oracle of the Spissa attention path -- TEST INFRASTRUCTURE ONLY.

A ctypes wrapper over oracle/_build/libspissa_oracle.so, the C restatement of
crates/spissa-runtime/src/rotary.rs:6-599, ops.rs:62-105 and 159-291, and the
weight decoding of tensor.rs and streaming/mod.rs (see
spissa_oracle.c for per-function citations). Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import this package, and only as the
checker or the timed CPU baseline. spissa_amd never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libspissa_oracle.so"

OK, SHAPE, INVALID = 0, 1, 2


class OracleError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code
        self.kind = {SHAPE: "Shape", INVALID: "InvalidTensorData"}.get(code, "Error")


class RotCfg(C.Structure):
    _fields_ = [("seq_len", C.c_size_t), ("num_heads", C.c_size_t), ("head_dim", C.c_size_t),
                ("rotary_dim", C.c_size_t), ("base", C.c_float), ("position_offset", C.c_size_t)]


class AttnCfg(C.Structure):
    _fields_ = [("query_len", C.c_size_t), ("num_heads", C.c_size_t), ("kv_heads", C.c_size_t),
                ("head_dim", C.c_size_t), ("causal", C.c_int), ("window", C.c_size_t)]


class KvC(C.Structure):
    _fields_ = [("num_heads", C.c_size_t), ("head_dim", C.c_size_t), ("max_seq_len", C.c_size_t),
                ("len", C.c_size_t), ("keys", C.POINTER(C.c_float)),
                ("values", C.POINTER(C.c_float))]


_lib = None
_fp = C.POINTER(C.c_float)
_sz = C.c_size_t


def build() -> Path:
    """Compiles the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def load() -> C.CDLL:
    """Loads the oracle library; SPISSA_ORACLE_LIB names another build of the
    same sources (the Makefile's `asan` target, for a sanitizer run)."""
    global _lib
    if _lib is not None:
        return _lib
    alt = os.environ.get("SPISSA_ORACLE_LIB")
    if alt:
        lib = C.CDLL(alt)
    else:
        if not LIB_PATH.exists():
            build()
        lib = C.CDLL(str(LIB_PATH))
    sig = {
        "or_last_error": (C.c_char_p, []),
        "or_gpt_neox_rotary_dim": (C.c_int, [_sz, C.c_float, C.POINTER(_sz)]),
        "or_apply_gpt_neox_rotary_inplace": (C.c_int, [_fp, _sz, _fp, _sz, C.POINTER(RotCfg)]),
        "or_apply_llama_rotary_inplace": (C.c_int, [_fp, _sz, _fp, _sz, _sz, _sz, C.POINTER(RotCfg), _fp, _sz]),
        "or_apply_gemma_rotary_inplace": (C.c_int, [_fp, _sz, _fp, _sz, _sz, _sz, C.POINTER(RotCfg), C.c_float]),
        "or_llama_cos_sin": (None, [_sz, _sz, _sz, C.c_float, C.c_float, _fp, _fp]),
        "or_gemma_cos_sin": (None, [_sz, _sz, _sz, C.c_float, C.c_float, _fp, _fp]),
        "or_kv_new": (C.POINTER(KvC), [_sz, _sz, _sz, C.POINTER(C.c_int)]),
        "or_kv_free": (None, [C.POINTER(KvC)]),
        "or_kv_append": (C.c_int, [C.POINTER(KvC), _fp, _sz, _fp, _sz, _sz]),
        "or_kv_clear": (None, [C.POINTER(KvC)]),
        "or_kv_truncate": (C.c_int, [C.POINTER(KvC), _sz]),
        "or_kv_resident_bytes": (_sz, [C.POINTER(KvC)]),
        "or_kv_len": (_sz, [C.POINTER(KvC)]),
        "or_sdpa_with_cache": (C.c_int, [_fp, _sz, _fp, _sz, _fp, _sz, C.POINTER(KvC), C.POINTER(AttnCfg), _fp, _sz]),
        "or_rms_norm": (C.c_int, [_fp, _sz, _fp, _sz, _sz, _sz, C.c_float, _fp]),
        "or_softmax_rows": (C.c_int, [_fp, _sz, _sz, _sz, _fp]),
        "or_scaled_dot_product_attention": (C.c_int, [_fp, _fp, _fp, _sz, _sz, _sz, _sz, C.c_int, _fp]),
        "or_is_global_layer": (C.c_int, [_sz, _sz]),
        "or_gemma_qk_prologue": (C.c_int, [_fp, _sz, _fp, _sz, _sz, _sz, _sz, _sz, _fp, _fp, C.c_float,
                                           C.c_float, C.c_float, _sz, C.c_float]),
        "or_bf16_to_f32": (C.c_float, [C.c_uint16]),
        "or_fp16_to_f32": (C.c_float, [C.c_uint16]),
        "or_f32_to_bf16_rne": (C.c_uint16, [C.c_float]),
        "or_linear": (C.c_int, [_fp, _sz, C.c_void_p, C.c_int, _sz, _fp, _sz, _sz, _sz, _sz, _fp]),
        "or_lm_head_logits": (C.c_int, [_fp, _sz, C.c_void_p, C.c_int, _sz, _sz, _fp]),
        "or_sample_argmax": (C.c_int, [_fp, _sz, C.POINTER(_sz)]),
        "or_sample_argmax_excluding": (C.c_int, [_fp, _sz, C.c_int, _sz, C.POINTER(_sz)]),
        "or_sdpa_many_threads": (C.c_int, [_sz, C.POINTER(_fp), C.POINTER(_fp), C.POINTER(_fp),
                                           C.POINTER(C.POINTER(KvC)), C.POINTER(AttnCfg),
                                           C.POINTER(_fp), C.c_int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _lib = lib
    return lib


def _check(code: int) -> None:
    if code != OK:
        raise OracleError(code, load().or_last_error().decode())


def _p(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def gpt_neox_rotary_dim(head_dim: int, pct: float) -> int:
    out = _sz()
    _check(load().or_gpt_neox_rotary_dim(head_dim, pct, C.byref(out)))
    return out.value


def apply_gpt_neox_rotary_inplace(q, k, seq_len, num_heads, head_dim, rotary_dim, base, offset):
    cfg = RotCfg(seq_len, num_heads, head_dim, rotary_dim, base, offset)
    _check(load().or_apply_gpt_neox_rotary_inplace(_p(q), q.size, _p(k), k.size, C.byref(cfg)))


def apply_llama_rotary_inplace(q, k, q_heads, k_heads, seq_len, head_dim, rotary_dim, base, offset,
                               freq_scale=None):
    cfg = RotCfg(seq_len, q_heads, head_dim, rotary_dim, base, offset)
    _check(load().or_apply_llama_rotary_inplace(_p(q), q.size, _p(k), k.size, q_heads, k_heads,
                                                C.byref(cfg), _p(freq_scale),
                                                0 if freq_scale is None else freq_scale.size))


def apply_gemma_rotary_inplace(q, k, q_heads, k_heads, seq_len, head_dim, rotary_dim, base, offset,
                               divisor):
    cfg = RotCfg(seq_len, q_heads, head_dim, rotary_dim, base, offset)
    _check(load().or_apply_gemma_rotary_inplace(_p(q), q.size, _p(k), k.size, q_heads, k_heads,
                                                C.byref(cfg), divisor))


class KvCache:
    """rotary.rs:195-318 on the CPU."""

    def __init__(self, num_heads: int, head_dim: int, max_seq_len: int):
        st = C.c_int()
        self._c = load().or_kv_new(num_heads, head_dim, max_seq_len, C.byref(st))
        _check(st.value)
        self.num_heads, self.head_dim = num_heads, head_dim

    def __del__(self):
        if getattr(self, "_c", None):
            load().or_kv_free(self._c)
            self._c = None

    def append(self, keys, values, n):
        _check(load().or_kv_append(self._c, _p(keys), keys.size, _p(values), values.size, n))

    def clear(self):
        load().or_kv_clear(self._c)

    def truncate(self, n):
        _check(load().or_kv_truncate(self._c, n))

    def len(self) -> int:
        return load().or_kv_len(self._c)

    def resident_bytes(self) -> int:
        return load().or_kv_resident_bytes(self._c)

    def keys(self) -> np.ndarray:
        n = self.len() * self.num_heads * self.head_dim
        return np.ctypeslib.as_array(self._c.contents.keys, shape=(max(n, 1),))[:n].copy()

    def values(self) -> np.ndarray:
        n = self.len() * self.num_heads * self.head_dim
        return np.ctypeslib.as_array(self._c.contents.values, shape=(max(n, 1),))[:n].copy()


def sdpa_with_cache(q, k, v, cache: Optional[KvCache], query_len, num_heads, kv_heads, head_dim,
                    causal=True, window=0) -> np.ndarray:
    cfg = AttnCfg(query_len, num_heads, kv_heads, head_dim, 1 if causal else 0, window)
    out = np.empty(q.size, dtype=np.float32)
    _check(load().or_sdpa_with_cache(_p(q), q.size, _p(k), k.size, _p(v), v.size,
                                     None if cache is None else cache._c, C.byref(cfg), _p(out), out.size))
    return out


def sdpa_many(units, cfg_tuple, threads: int):
    """Runs sdpa_with_cache over [(q, k, v, cache)] units on `threads` POSIX threads."""
    n = len(units)
    qa = (_fp * n)(*[_p(u[0]) for u in units])
    ka = (_fp * n)(*[_p(u[1]) for u in units])
    va = (_fp * n)(*[_p(u[2]) for u in units])
    ca = (C.POINTER(KvC) * n)(*[u[3]._c if u[3] is not None else C.POINTER(KvC)() for u in units])
    outs = [np.empty(u[0].size, dtype=np.float32) for u in units]
    oa = (_fp * n)(*[_p(o) for o in outs])
    cfg = AttnCfg(*cfg_tuple)
    _check(load().or_sdpa_many_threads(n, qa, ka, va, ca, C.byref(cfg), oa, threads))
    return outs


def rms_norm(x, w, rows, cols, eps) -> np.ndarray:
    out = np.empty(x.size, dtype=np.float32)
    _check(load().or_rms_norm(_p(x), x.size, _p(w), w.size, rows, cols, eps, _p(out)))
    return out


def softmax_rows(logits, rows, cols) -> np.ndarray:
    out = np.empty(logits.size, dtype=np.float32)
    _check(load().or_softmax_rows(_p(logits), logits.size, rows, cols, _p(out)))
    return out


def scaled_dot_product_attention(q, k, v, seq_len, num_heads, head_dim, causal) -> np.ndarray:
    out = np.empty(q.size, dtype=np.float32)
    _check(load().or_scaled_dot_product_attention(_p(q), _p(k), _p(v), q.size, seq_len, num_heads,
                                                  head_dim, 1 if causal else 0, _p(out)))
    return out


def is_global_layer(layer, pattern) -> bool:
    return bool(load().or_is_global_layer(layer, pattern))


def gemma_qk_prologue(q, k, seq_len, q_heads, kv_heads, head_dim, q_norm, k_norm, eps, base,
                      divisor, offset, qpas):
    _check(load().or_gemma_qk_prologue(_p(q), q.size, _p(k), k.size, seq_len, q_heads, kv_heads,
                                       head_dim, _p(q_norm), _p(k_norm), eps, base, divisor, offset,
                                       qpas))


def llama_cos_sin(pos, pair, rotary_dim, base, freq_scale=1.0):
    c, s = C.c_float(), C.c_float()
    load().or_llama_cos_sin(pos, pair, rotary_dim, base, freq_scale, C.byref(c), C.byref(s))
    return c.value, s.value


DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2


def bf16_to_f32(bits: int) -> float:
    return load().or_bf16_to_f32(bits)


def fp16_to_f32(bits: int) -> float:
    return load().or_fp16_to_f32(bits)


def f32_to_bf16_rne(x: float) -> int:
    return load().or_f32_to_bf16_rne(x)


def linear(x, w, dtype, bias, batch, in_features, out_features) -> np.ndarray:
    """ops.rs:62-105 over the decoded weight. w: float32 array (DTYPE_F32) or
    uint16 array of bf16 / binary16 bits, [out, in] row-major."""
    want = np.float32 if dtype == DTYPE_F32 else np.uint16
    assert w.dtype == want and w.flags.c_contiguous
    out = np.empty(batch * out_features, dtype=np.float32)
    _check(load().or_linear(_p(x), x.size, w.ctypes.data_as(C.c_void_p), dtype, w.size, _p(bias),
                            0 if bias is None else bias.size, batch, in_features, out_features, _p(out)))
    return out


def lm_head_logits(last_hidden, table, dtype, vocab_size, hidden) -> np.ndarray:
    """streaming/mod.rs:186-287 (serial row loop). table: float32 (DTYPE_F32)
    or uint16 bf16 bits (DTYPE_BF16), [vocab_size, hidden] row-major."""
    want = np.float32 if dtype == DTYPE_F32 else np.uint16
    assert table.dtype == want and table.flags.c_contiguous and table.size == vocab_size * hidden
    out = np.empty(vocab_size, dtype=np.float32)
    _check(load().or_lm_head_logits(_p(last_hidden), last_hidden.size, table.ctypes.data_as(C.c_void_p),
                                    dtype, vocab_size, hidden, _p(out)))
    return out


def sample_argmax(logits) -> int:
    """ops.rs:309-324"""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    r = _sz(0)
    _check(load().or_sample_argmax(_p(x), x.size, C.byref(r)))
    return r.value


def sample_argmax_excluding(logits, excluded: Optional[int]) -> int:
    """ops.rs:326-348"""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    r = _sz(0)
    _check(load().or_sample_argmax_excluding(_p(x), x.size, 0 if excluded is None else 1,
                                             0 if excluded is None else excluded, C.byref(r)))
    return r.value

