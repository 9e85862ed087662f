"""Weight formats, quantized tensors and the matmul / quantize dispatch.

Python mirror of the reference's `weight_type.rs` public surface
(weight_type.rs:17-120) over the HIP implementation:
  WeightFormat            weight_type.rs:17-22
  QuantizedWeight         QuantizedTensor::{Q8,Q4_0} (weight_type.rs:30-50),
                          resident on the device
  quantize(fmt, x)        weight_type::quantize (weight_type.rs:76-90)
  matmul(out, x, w, ...)  weight_type::matmul (weight_type.rs:92-106)
Format mismatches raise (the reference panics, weight_type.rs:88,104).
"""
from __future__ import annotations

import enum

import numpy as np

from ._lib import YlError, check, last_error, lib
from .device import DeviceBuffer


class WeightFormat(enum.IntEnum):
    Q8_0 = 0
    Q4_0 = 1
    F16 = 2


class QuantizedWeight:
    """A quantized [o][n] matrix on the device."""

    def __init__(self, handle, fmt: WeightFormat, o: int, n: int):
        self._h = handle
        self.fmt = WeightFormat(fmt)
        self.o, self.n = int(o), int(n)

    @classmethod
    def upload(cls, fmt: WeightFormat, quant_vals: np.ndarray, scale_factor: np.ndarray, o: int, n: int):
        """From the reference's in-memory form (Q4_0: nibble values 0..15 per element)."""
        q = np.ascontiguousarray(quant_vals, np.int8)
        s = np.ascontiguousarray(scale_factor, np.float32)
        if q.size != o * n or s.size != o * n // 32:
            raise ValueError("quant_vals must hold o*n values and scale_factor o*n/32")
        h = lib().yl_weight_upload(int(fmt), q.ctypes.data, s.ctypes.data, o, n)
        if not h:
            raise YlError(-1, last_error())
        return cls(h, fmt, o, n)

    @classmethod
    def upload_gguf(cls, fmt: WeightFormat, blocks: bytes | np.ndarray, o: int, n: int):
        """From raw GGUF Q8_0 (34-byte) / Q4_0 (18-byte) blocks."""
        b = np.frombuffer(bytes(blocks), np.uint8) if not isinstance(blocks, np.ndarray) else blocks
        b = np.ascontiguousarray(b, np.uint8)
        per = 34 if fmt == WeightFormat.Q8_0 else 18
        if b.size != o * n // 32 * per:
            raise ValueError("block buffer size does not match o*n")
        h = lib().yl_weight_upload_gguf(int(fmt), b.ctypes.data, o, n)
        if not h:
            raise YlError(-1, last_error())
        return cls(h, fmt, o, n)

    @classmethod
    def upload_f16(cls, values: np.ndarray, o: int, n: int):
        """QuantizedTensor::F16 from float16 values (or their bits as uint16)."""
        v = np.ascontiguousarray(values)
        bits = v.view(np.uint16) if v.dtype == np.float16 else np.ascontiguousarray(v, np.uint16)
        if bits.size != o * n:
            raise ValueError("values must hold o*n elements")
        h = lib().yl_weight_upload_f16(bits.ctypes.data, o, n)
        if not h:
            raise YlError(-1, last_error())
        return cls(h, WeightFormat.F16, o, n)

    @property
    def nbytes(self) -> int:
        return int(lib().yl_weight_bytes(self._h))

    def free(self):
        if self._h:
            lib().yl_weight_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def quantize_device(fmt: WeightFormat, q: DeviceBuffer, s: DeviceBuffer, x: DeviceBuffer, n: int, gs: int = 32,
                    stream=None) -> None:
    check(lib().yl_quantize(int(fmt), q.ptr, s.ptr, x.ptr, n, gs, stream))


def quantize(fmt: WeightFormat, x: np.ndarray, gs: int = 32):
    """Quantize host floats on the device -> (int8 values, f32 scales) on the host."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    dx = DeviceBuffer.from_numpy(x)
    dq = DeviceBuffer.zeros(x.size, np.int8)
    ds = DeviceBuffer.zeros(max(1, x.size // gs), np.float32)
    quantize_device(fmt, dq, ds, dx, x.size, gs)
    return dq.numpy(), ds.numpy()[: x.size // gs]


def matmul_device(out: DeviceBuffer, fmt: WeightFormat, xq: DeviceBuffer, xs: DeviceBuffer, batch: int,
                  w: QuantizedWeight, n: int, o: int, gs: int = 32, stream=None) -> None:
    check(lib().yl_matmul(out.ptr, int(fmt), xq.ptr, xs.ptr, batch, w._h, n, o, gs, stream))


def matmul(out: np.ndarray, x_q: np.ndarray, x_scale: np.ndarray, w: QuantizedWeight, n: int, o: int,
           gs: int = 32, fmt: WeightFormat | None = None) -> np.ndarray:
    """weight_type::matmul with host arrays: `out` (batch*o) is updated like the
    reference (`+=` for the first 4*floor(o/4) columns, `=` for the rest)."""
    batch = out.size // o
    dout = DeviceBuffer.from_numpy(np.ascontiguousarray(out, np.float32))
    dq = DeviceBuffer.from_numpy(np.ascontiguousarray(x_q, np.int8))
    ds = DeviceBuffer.from_numpy(np.ascontiguousarray(x_scale, np.float32))
    matmul_device(dout, w.fmt if fmt is None else fmt, dq, ds, batch, w, n, o, gs)
    out[...] = dout.numpy().reshape(out.shape)
    return out


def matmul_f32(x: np.ndarray, w: QuantizedWeight, n: int, o: int) -> np.ndarray:
    """matmul_f32 (weight_type.rs:228-270) on an F16 weight: x [batch][n] f32 ->
    [batch][o], every column assigned."""
    x = np.ascontiguousarray(x, np.float32)
    batch = x.size // n
    dx = DeviceBuffer.from_numpy(x.ravel())
    dout = DeviceBuffer.zeros(batch * o, np.float32)
    check(lib().yl_matmul_f32(dout.ptr, dx.ptr, batch, w._h, n, o, None))
    return dout.numpy().reshape(batch, o)
