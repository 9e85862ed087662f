"""Per-op entry points of the forward path on host arrays (device compute).

Each wraps one C-ABI op so tests can compare it with the reference function
it mirrors:
  rmsnorm_quantize  util::rmsnorm (util.rs:389-426) + quantize
  rope_gguf         util::rope_gguf (util.rs:653-718)
  attention         forward.rs fused_attention (forward.rs:299-400)
  swiglu_quantize   forward.rs:220-237 + quantize
  math_selftest     device exp / sqrt / division / f16 widening probes
  serial_sum_selftest  the one-wavefront exact serial f32 sum (softmax denominator)
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import RopeParams, check, lib
from .device import DeviceBuffer


def rmsnorm_quantize(x: np.ndarray, weight: np.ndarray, eps: float, qfmt: int = -1):
    """Rows of x [batch][size] -> (normalized f32, q int8 or None, scales or None)."""
    x = np.ascontiguousarray(x, np.float32)
    batch, size = (1, x.size) if x.ndim == 1 else x.shape
    dx, dw = DeviceBuffer.from_numpy(x), DeviceBuffer.from_numpy(np.ascontiguousarray(weight, np.float32))
    dn = DeviceBuffer.zeros(x.size, np.float32)
    dq = DeviceBuffer.zeros(max(1, x.size), np.int8)
    ds = DeviceBuffer.zeros(max(1, x.size // 32), np.float32)
    check(lib().yl_rmsnorm_quantize(dx.ptr, dw.ptr, size, eps, batch, dn.ptr, qfmt, dq.ptr if qfmt >= 0 else None,
                                    ds.ptr if qfmt >= 0 else None, None))
    check(lib().yl_synchronize())
    xn = dn.numpy().reshape(x.shape)
    if qfmt < 0:
        return xn, None, None
    return xn, dq.numpy()[: x.size], ds.numpy()[: x.size // 32]


def rope_gguf(params: RopeParams, q: np.ndarray, k: np.ndarray, start_pos: int, batch: int = 1):
    dq = DeviceBuffer.from_numpy(np.ascontiguousarray(q, np.float32))
    dk = DeviceBuffer.from_numpy(np.ascontiguousarray(k, np.float32))
    check(lib().yl_rope_gguf(C.byref(params), dq.ptr, dk.ptr, batch, start_pos, None))
    return dq.numpy().reshape(np.shape(q)), dk.numpy().reshape(np.shape(k))


def attention(q: np.ndarray, key_cache: np.ndarray, value_cache: np.ndarray, batch: int, start_pos: int,
              n_heads: int, n_kv_heads: int, head_size: int, attn_scale: float) -> np.ndarray:
    dq = DeviceBuffer.from_numpy(np.ascontiguousarray(q, np.float32))
    dk = DeviceBuffer.from_numpy(np.ascontiguousarray(key_cache, np.float32))
    dv = DeviceBuffer.from_numpy(np.ascontiguousarray(value_cache, np.float32))
    out = DeviceBuffer.zeros(batch * n_heads * head_size, np.float32)
    check(lib().yl_attention(out.ptr, dq.ptr, dk.ptr, dv.ptr, batch, start_pos, n_heads, n_kv_heads, head_size,
                             attn_scale, None))
    return out.numpy()


def attention_split(q: np.ndarray, key_cache: np.ndarray, value_cache: np.ndarray, start_pos: int,
                    n_heads: int, n_kv_heads: int, head_size: int, attn_scale: float) -> np.ndarray:
    """The split decode attention (one query row at start_pos): equal to
    fused_attention (forward.rs:299-400) up to rounding."""
    dq = DeviceBuffer.from_numpy(np.ascontiguousarray(q, np.float32))
    dk = DeviceBuffer.from_numpy(np.ascontiguousarray(key_cache, np.float32))
    dv = DeviceBuffer.from_numpy(np.ascontiguousarray(value_cache, np.float32))
    out = DeviceBuffer.zeros(n_heads * head_size, np.float32)
    check(lib().yl_attention_split(out.ptr, dq.ptr, dk.ptr, dv.ptr, start_pos, n_heads, n_kv_heads, head_size,
                                   attn_scale, None))
    return out.numpy()


def swiglu_quantize(gate: np.ndarray, up: np.ndarray, qfmt: int = -1):
    g = np.ascontiguousarray(gate, np.float32)
    batch, hidden = (1, g.size) if g.ndim == 1 else g.shape
    dg, du = DeviceBuffer.from_numpy(g), DeviceBuffer.from_numpy(np.ascontiguousarray(up, np.float32))
    dh = DeviceBuffer.zeros(g.size, np.float32)
    dq = DeviceBuffer.zeros(max(1, g.size), np.int8)
    ds = DeviceBuffer.zeros(max(1, g.size // 32), np.float32)
    check(lib().yl_swiglu_quantize(dg.ptr, du.ptr, hidden, batch, dh.ptr, qfmt, dq.ptr if qfmt >= 0 else None,
                                   ds.ptr if qfmt >= 0 else None, None))
    check(lib().yl_synchronize())
    h = dh.numpy().reshape(g.shape)
    if qfmt < 0:
        return h, None, None
    return h, dq.numpy()[: g.size], ds.numpy()[: g.size // 32]


def math_selftest(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    dx = DeviceBuffer.from_numpy(x)
    outs = [DeviceBuffer.zeros(x.size, np.float32) for _ in range(4)]
    check(lib().yl_math_selftest(dx.ptr, x.size, *[o.ptr for o in outs]))
    return tuple(o.numpy() for o in outs)


def serial_sum_selftest(segments, piece: int = 0):
    """Device serial f32 sums ((0 + v0) + v1) + ... of each nonnegative segment
    (piece > 0: summed in consecutive pieces of that many values, each piece
    continuing from the previous one's sum; piece -1: by the decode
    attention's segmented sum over four wavefronts; piece -2: by the
    long-context softmax's wide segmented sum over eight wavefronts)."""
    segs = [np.ascontiguousarray(s, np.float32).ravel() for s in segments]
    offs = np.zeros(len(segs) + 1, np.uint32)
    offs[1:] = np.cumsum([s.size for s in segs])
    v = np.concatenate(segs) if segs else np.zeros(1, np.float32)
    dv, do = DeviceBuffer.from_numpy(v if v.size else np.zeros(1, np.float32)), DeviceBuffer.from_numpy(offs)
    out = DeviceBuffer.zeros(max(1, len(segs)), np.float32)
    check(lib().yl_serial_sum_selftest(dv.ptr, do.ptr, len(segs), int(piece) & 0xFFFFFFFF, out.ptr))
    return out.numpy()[: len(segs)]
