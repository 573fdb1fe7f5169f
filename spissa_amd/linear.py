"""Host-side mirror of the streaming linear projection with the weight
resident in HBM: crates/spissa-runtime/src/streaming/linear.rs:269-576
(streaming_tile_linear_from_model) and streaming/mod.rs:511-526
(StreamingLinearConfig, StreamingTileLinearConfig).

The reference streams each weight out of the model container chunk by chunk
on every call. Here a `LinearWeight` uploads the weight's raw element bytes
once; a `LinearModel` maps tensor names to resident weights and stands where
the reference's `LazySpissaModel` does. The arithmetic is
out[batch, out] = input[batch, in] x W[out, in]^T + bias (ops.rs:62-105), in
f32, on the GPU.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np

from . import _ffi
from .errors import ArgumentError, ShapeError, SpissaError, check
from .rotary import _f32, _ptr

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2


class MissingTensorError(SpissaError):
    """RuntimeError::MissingTensor (lazy.rs:357-361)."""

    kind = "MissingTensor"


@dataclass(frozen=True)
class StreamingLinearConfig:
    """streaming/mod.rs:511-516"""

    batch: int
    in_features: int
    out_features: int

    def _c(self) -> _ffi.LinearConfigC:
        return _ffi.LinearConfigC(self.batch, self.in_features, self.out_features)


@dataclass(frozen=True)
class StreamingTileLinearConfig:
    """streaming/mod.rs:518-526. tile_elements bounds the reference's f32 CPU
    scratch; the device path has no such scratch, so it is only validated."""

    linear: StreamingLinearConfig
    tile_elements: int


class LinearWeight:
    """A [out_features, in_features] weight resident in HBM.

    data: float32 array (DTYPE_F32) or uint16 array of bf16 / binary16 bits
    (DTYPE_BF16 / DTYPE_F16), row-major, out_features * in_features elements;
    or a contiguous device tensor of the same bytes (float32, or a 16-bit
    dtype), copied device to device after the current stream's work.
    """

    def __init__(self, data, dtype: int, out_features: int, in_features: int, session=None):
        lib = _ffi.load()
        self._lib = lib
        if getattr(data, "is_cuda", False):
            import torch

            ok = data.dtype == torch.float32 if dtype == DTYPE_F32 else data.element_size() == 2
            if not ok or not data.is_contiguous():
                raise TypeError("device weight data must be a contiguous tensor of the dtype's width")
            torch.cuda.current_stream(data.device).synchronize()
            ptr, nbytes = _ffi.c_void_p(data.data_ptr()), data.numel() * data.element_size()
        else:
            want = np.float32 if dtype == DTYPE_F32 else np.uint16
            if data.dtype != want or not data.flags.c_contiguous:
                raise TypeError(f"weight data must be a contiguous {np.dtype(want).name} array")
            ptr, nbytes = data.ctypes.data_as(_ffi.c_void_p), data.nbytes
        s = session.handle if session is not None else self._default_session(lib)
        # the weight is freed through its session: keep the session alive as long
        self._session = session
        h = _ffi.c_void_p()
        check(lib.spissa_linear_weight_new(s, dtype, out_features, in_features, ptr, nbytes, C.byref(h)))
        self._h = h
        self.dtype, self.out_features, self.in_features = dtype, out_features, in_features

    @staticmethod
    def _default_session(lib):
        s = _ffi.c_void_p()
        check(lib.spissa_default_session(C.byref(s)))
        return s

    @property
    def handle(self):
        if self._h is None or not self._h.value:
            raise ArgumentError("LinearWeight has been closed")
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            self._lib.spissa_linear_weight_free(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class LinearModel:
    """Resident weights by tensor name (the role of lazy.rs's LazySpissaModel)."""

    def __init__(self, weights: Optional[Dict[str, LinearWeight]] = None):
        self._w: Dict[str, LinearWeight] = dict(weights or {})

    def add(self, name: str, weight: LinearWeight) -> None:
        self._w[name] = weight

    def tensor(self, name: str) -> LinearWeight:
        """lazy.rs:357-361"""
        try:
            return self._w[name]
        except KeyError:
            raise MissingTensorError(name) from None


def linear(weight: LinearWeight, input: np.ndarray, bias: Optional[np.ndarray],
           config: StreamingLinearConfig) -> np.ndarray:
    """input[batch, in] x W^T + bias on the GPU; validation as
    streaming/validation.rs:225-289 (Shape errors)."""
    _f32(input, "input")
    if bias is not None:
        _f32(bias, "bias")
    out = np.empty(config.batch * config.out_features, dtype=np.float32)
    cfg = config._c()
    check(_ffi.load().spissa_linear(weight.handle, _ptr(input), input.size, _ptr(bias),
                                    0 if bias is None else bias.size, C.byref(cfg), _ptr(out),
                                    out.size))
    return out


def streaming_tile_linear_from_model(model: LinearModel, weight_name: str, input: np.ndarray,
                                     bias: Optional[np.ndarray],
                                     config: StreamingTileLinearConfig) -> np.ndarray:
    """streaming/linear.rs:269-576 with the weight already in HBM."""
    if config.tile_elements == 0:  # streaming/validation.rs:249-256
        raise ShapeError("tile_elements must be greater than zero")
    w = model.tensor(weight_name)
    return linear(w, input, bias, config.linear)
