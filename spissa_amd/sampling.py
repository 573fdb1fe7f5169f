"""Host-side mirror of the LM head and greedy sampling:
crates/spissa-runtime/src/streaming/mod.rs:186-287 (lm_head_logits_parallel,
lm_head_logits_parallel_bf16) and ops.rs:309-348 (sample_argmax,
sample_argmax_excluding).

The reference reads the tied embedding table from the model container on
every call. Here the table is a `LinearWeight` of shape [vocab_size, hidden]
resident in HBM, and `vocab_size` / `hidden` are checked against it. The
argmax runs on the GPU and reproduces the reference's sequential scan,
including its tie and NaN behaviour.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional

import numpy as np

from . import _ffi
from .errors import ShapeError, check
from .linear import DTYPE_BF16, DTYPE_F32, LinearWeight
from .rotary import _f32, _ptr


def _logits(table: LinearWeight, last_hidden: np.ndarray, vocab_size: int, hidden: int,
            dtype: int) -> np.ndarray:
    _f32(last_hidden, "last_hidden")
    if table.dtype != dtype:
        raise TypeError("table dtype does not match this LM head variant")
    if table.out_features != vocab_size or table.in_features != hidden:
        raise ShapeError(f"table is [{table.out_features}, {table.in_features}], requested "
                         f"[{vocab_size}, {hidden}]")
    out = np.empty(vocab_size, dtype=np.float32)
    check(_ffi.load().spissa_lm_head_logits(table.handle, _ptr(last_hidden), last_hidden.size,
                                            _ptr(out), out.size))
    return out


def lm_head_logits_parallel(last_hidden: np.ndarray, table: LinearWeight, vocab_size: int,
                            hidden: int) -> np.ndarray:
    """streaming/mod.rs:186-221: logits[v] = sum_h last_hidden[h] * table[v, h], f32 table."""
    return _logits(table, last_hidden, vocab_size, hidden, DTYPE_F32)


def lm_head_logits_parallel_bf16(last_hidden: np.ndarray, table: LinearWeight, vocab_size: int,
                                 hidden: int) -> np.ndarray:
    """streaming/mod.rs:238-272, bf16 table."""
    return _logits(table, last_hidden, vocab_size, hidden, DTYPE_BF16)


def _session(session):
    if session is not None:
        return session.handle
    s = _ffi.c_void_p()
    check(_ffi.load().spissa_default_session(C.byref(s)))
    return s


def _argmax(logits, excluded: int, session) -> int:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    tok = _ffi.c_size(0)
    check(_ffi.load().spissa_sample_argmax(_session(session), _ptr(x), x.size, excluded, C.byref(tok)))
    return tok.value


def sample_argmax(logits, session=None) -> int:
    """ops.rs:309-324: the first index of the maximum; empty logits raise
    InvalidTensorDataError."""
    return _argmax(logits, -1, session)


def sample_argmax_excluding(logits, excluded_token: Optional[int], session=None) -> int:
    """ops.rs:326-348: the argmax with `excluded_token` skipped (None, an index
    past the end, or a single logit: plain sample_argmax)."""
    if excluded_token is not None and excluded_token < 0:
        raise ValueError("excluded_token is an index (usize)")
    return _argmax(logits, -1 if excluded_token is None else excluded_token, session)
