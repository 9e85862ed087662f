"""CPU model of the device's one-wavefront serial sum (wave_serial_sum in
csrc/yl_device.h), round by round, held to the sequential f32 loop it
replaces: while the running sum s stays in one binade it is a multiple of
that binade's ulp u, so a step adds v rounded to a multiple of u unless v/u
is an exact tie; each round takes 64 values as integers, prefix-sums them
and stops at the first tie, binade exit, or value that leaves the binade."""
import numpy as np

from serial_sum_cases import cases, sequential

F = np.float32


def model_sum(v):
    v = np.asarray(v, F)
    n, s, t = v.size, F(0.0), 0
    while t < n:
        lanes = np.zeros(64, F)
        k_ = min(64, n - t)
        lanes[:k_] = v[t:t + k_]
        if s == 0:
            nz = np.nonzero(lanes != 0)[0]
            if nz.size == 0:
                t += 64
                continue
            s = lanes[nz[0]]
            t += int(nz[0]) + 1
            continue
        ex = int(np.frexp(s)[1])
        k = max(ex - 24, -149)
        B = F(np.ldexp(1.0, ex)) if ex - 1 >= -126 else F(2.0 ** -126)
        bad = ~(lanes < B)
        with np.errstate(over="ignore", invalid="ignore"):   # only lanes already marked bad overflow
            q = np.ldexp(lanes, -k).astype(F)
            r = np.rint(q).astype(F)
            bad |= np.abs(q - r) == F(0.5)
        pre = np.cumsum(np.where(bad, F(0), r), dtype=F)   # exact: integers < 2^24
        cand = (s + np.ldexp(pre, k).astype(F)).astype(F)
        bad |= ~(cand < B)
        if not bad.any():
            s = cand[63]
            t += 64
        else:
            L = int(np.argmax(bad))
            sp = cand[L - 1] if L > 0 else s
            s = F(sp + lanes[L])
            t += L + 1
    return s


def test_model_equals_sequential_sum():
    for v in cases(seed=1, count=70, max_len=3000):
        a, b = sequential(v), model_sum(v)
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), (v.size, a, b)


def test_model_ties_and_binade_edges():
    # values landing exactly on half-ulp ties of a sum just below a power of two
    v = np.array([1.0, 0.5, 0.25] + [2.0 ** -24] * 40 + [3 * 2.0 ** -25] * 40 + [1.0 - 2.0 ** -24] * 30, F)
    assert sequential(v).view(np.uint32) == model_sum(v).view(np.uint32)
