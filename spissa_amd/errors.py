"""Error types of the attention path.

They mirror the RuntimeError variants the reference returns from this path
(crates/spissa-runtime/src/error.rs:6-54): Shape and InvalidTensorData. Device
and argument failures have no reference counterpart.
"""
from __future__ import annotations

from . import _ffi


class SpissaError(RuntimeError):
    """Base class; `kind` is the reference variant name."""

    kind = "Error"


class ShapeError(SpissaError):
    """RuntimeError::Shape (error.rs:12)."""

    kind = "Shape"


class InvalidTensorDataError(SpissaError):
    """RuntimeError::InvalidTensorData (error.rs:24)."""

    kind = "InvalidTensorData"


class DeviceError(SpissaError):
    """A HIP runtime failure."""

    kind = "Device"


class ArgumentError(SpissaError):
    """A null handle or buffer passed across the C boundary."""

    kind = "Argument"


_BY_CODE = {
    _ffi.ERR_SHAPE: ShapeError,
    _ffi.ERR_INVALID_TENSOR_DATA: InvalidTensorDataError,
    _ffi.ERR_DEVICE: DeviceError,
    _ffi.ERR_ARGUMENT: ArgumentError,
}


def check(status: int) -> None:
    """Raises the exception matching a non-zero status of the C ABI."""
    if status == _ffi.OK:
        return
    cls = _BY_CODE.get(status, SpissaError)
    raise cls(_ffi.last_error())
