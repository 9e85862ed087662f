"""CPU model of the device's segmented serial sum (seg_serial_sum and
seg_serial_sum_wide in yallma3_mini_inference_amd/csrc/yl_blocks.h): the
softmax denominator ((0 + v0) + v1) + ... computed as segments summed from
candidate starts around a float64 estimate, then walked in order.

The model follows the device's index arithmetic (segment length, candidate
bases, the walk and the one-at-a-time fallback) and must equal the
sequential float32 loop bit for bit on every input; the drift bound that
makes the fast path the common one is checked on softmax-like rows."""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(__file__))
from serial_sum_cases import cases, sequential  # noqa: E402

f32 = np.float32


def _seg_len(n, ns):
    return 8 * -(-n // (8 * ns))


def _base(est, half):
    b = int(np.float32(est).view(np.int32)) - half
    return min(max(b, 0), 0x7F7FFFFF - 2 * half)


def _chain(start_bits, vals):
    s = np.array([start_bits], np.int32).view(np.float32)[0]
    for x in vals:
        s = f32(s + x)
    return s


def seg_sum(v, ns=8, cands=64):
    """The device's steps: ns segments, `cands` consecutive candidate starts
    each (64: seg_serial_sum; 128: seg_serial_sum_wide)."""
    v = np.asarray(v, np.float32)
    n = v.size
    if n == 0:
        return f32(0.0), 0
    L = _seg_len(n, ns)
    vp = np.zeros(ns * L, np.float32)
    vp[:n] = v
    assert ns * L <= 64 * -(-n // 64)            # within the +0 padding the callers write
    with np.errstate(all="ignore"):
        pre = np.concatenate([[0.0], np.cumsum([vp[i * L:(i + 1) * L].astype(np.float64).sum() for i in range(ns)])])
        bases = [0] + [_base(pre[i], cands // 2) for i in range(1, ns)]
        S = _chain(0, vp[:L])
        hits = 0
        for i in range(1, ns):
            if i * L >= n:
                break
            idx = int(np.float32(S).view(np.int32)) - bases[i]
            if 0 <= idx < cands:
                S = _chain(bases[i] + idx, vp[i * L:(i + 1) * L])   # the lane whose start is S
                hits += 1
            else:
                for k in range(i * L, n):
                    S = f32(S + vp[k])
                break
    return S, hits


def _same(a, b):
    return (np.isnan(a) and np.isnan(b)) or np.float32(a).view(np.int32) == np.float32(b).view(np.int32)


def test_model_exact_on_adversarial_rows():
    for v in cases(seed=5, count=30, max_len=2500):
        for ns, c in ((8, 64), (8, 128)):
            assert _same(seg_sum(v, ns, c)[0], sequential(v)), (v.size, ns, c)


def test_model_fallback_on_a_drifting_row():
    # after a first value of 1 every value is 3/4 ulp: each add rounds up by
    # 1/4 ulp, so the serial sum drifts 20 ulps per 80-value segment; the
    # walk takes segment 1 (20 ulps off), misses segment 2 (40 ulps off) and
    # continues one value at a time from there
    w = np.full(600, np.float32(0.75 * 2.0 ** -23), np.float32)
    w[0] = 1.0
    s, hits = seg_sum(w)
    assert hits == 1 and _same(s, sequential(w))


def test_softmax_rows_stay_within_the_window():
    rng = np.random.default_rng(1)
    worst = 0
    for t in range(60):
        n = int(rng.integers(300, 1025))
        x = rng.standard_normal(n).astype(np.float32) * rng.uniform(0.1, 3)
        e = np.exp((x - x.max()).astype(np.float64)).astype(np.float32)
        L = _seg_len(n, 8)
        ser = np.cumsum(e, dtype=np.float32)
        ex = np.cumsum(e.astype(np.float64))
        for i in range(1, 8):
            if i * L >= n:
                break
            d = int(ser[i * L - 1].view(np.int32)) - int(np.float32(ex[i * L - 1]).view(np.int32))
            worst = max(worst, abs(d))
        s, hits = seg_sum(e)
        assert _same(s, ser[-1])
    assert worst < 32, worst
