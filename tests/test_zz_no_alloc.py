"""yl_attention_noalloc against yl_attention through the C ABI.

The allocation-free entry point keeps its step state, transposed keys and
scores scratch in the library's per-GPU scratch array; its outputs must be
bit-identical to yl_attention's (which allocates those buffers per call) on
two calls in a row, the second smaller than the first, for the decode
kernels (one token: the split path of contexts beyond 4096 with its scores
scratch, and the single kernel) and the prompt kernels (tiled batches of 64+
tokens, and the one-row-per-workgroup kernel).  Calls whose buffers exceed
the array are refused with YL_ERR_RANGE before any work is enqueued.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _run(lib, fn, q, k, v, batch, start, nh, nkv, hd):
    from yallma3_mini_inference_amd import DeviceBuffer, check
    dq, dk, dv = DeviceBuffer.from_numpy(q), DeviceBuffer.from_numpy(k), DeviceBuffer.from_numpy(v)
    out = DeviceBuffer.zeros(batch * nh * hd, np.float32)
    check(fn(out.ptr, dq.ptr, dk.ptr, dv.ptr, batch, start, nh, nkv, hd, float(1.0 / np.sqrt(hd)), None))
    check(lib.yl_synchronize())
    return out.numpy()


# (first call, second smaller call): (batch, start_pos, n_heads, n_kv_heads, head_size)
PAIRS = [
    ((1, 8191, 32, 8, 128), (1, 699, 8, 2, 64)),      # split decode (scores scratch), then one kernel
    ((70, 30, 8, 2, 64), (20, 10, 8, 2, 64)),         # tiled prompt, then one row per workgroup
    ((1, 5000, 8, 2, 64), (1, 4500, 8, 2, 64)),       # split decode twice, shorter second
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_attention_noalloc_matches_attention(gpu, first, second):
    L = gpu.lib()
    rng = np.random.default_rng(sum(first) + sum(second))
    for batch, start, nh, nkv, hd in (first, second):
        seq = start + batch
        q = rng.standard_normal(batch * nh * hd, dtype=np.float32)
        k = rng.standard_normal(seq * nkv * hd, dtype=np.float32)
        v = rng.standard_normal(seq * nkv * hd, dtype=np.float32)
        ref = _run(L, L.yl_attention, q, k, v, batch, start, nh, nkv, hd)
        got = _run(L, L.yl_attention_noalloc, q, k, v, batch, start, nh, nkv, hd)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (batch, start, nh, nkv, hd)


def test_attention_noalloc_rejects_oversized_calls(gpu):
    from yallma3_mini_inference_amd import DeviceBuffer
    L = gpu.lib()
    nh, nkv, hd, seq = 32, 8, 128, 20000        # keys alone: 20000 * 1024 floats = 78 MiB
    dq = DeviceBuffer.zeros(nh * hd, np.float32)
    dkv = DeviceBuffer.zeros(8, np.float32)     # never read: the call is refused first
    out = DeviceBuffer.zeros(nh * hd, np.float32)
    st = L.yl_attention_noalloc(out.ptr, dq.ptr, dkv.ptr, dkv.ptr, 1, seq - 1, nh, nkv, hd, 0.088, None)
    assert st == -8
    assert b"scratch" in L.yl_last_error()
