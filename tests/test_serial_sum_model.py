"""CPU model of the device's one-wavefront serial sum (wave_serial_sum in
csrc/yl_device.h), row by row, held to the sequential f32 loop it replaces:
while the running sum s stays in one binade it is a multiple of that
binade's ulp u, so a step adds v rounded to a multiple of u unless v/u is an
exact tie; rows of 64 values are taken as integers and prefix-summed onto a
running total until the first tie, binade exit, or value that leaves the
binade, where one ordinary add restarts the binade."""
import numpy as np

from serial_sum_cases import cases, sequential

F = np.float32


def model_sum(v):
    v = np.asarray(v, F)
    n, s, t = v.size, F(0.0), 0
    while t < n:
        if s == 0:
            lanes = np.zeros(64, F)
            c = min(64, n - t)
            lanes[:c] = v[t:t + c]
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
        off = F(0.0)   # running total of the rows taken, in units of u
        while True:
            lanes = np.zeros(64, F)
            c = min(64, n - t)
            lanes[:c] = v[t:t + c]
            bad = ~(lanes < B)
            with np.errstate(over="ignore", invalid="ignore"):   # only lanes already marked bad overflow
                q = np.ldexp(lanes, -k).astype(F)
                r = np.rint(q).astype(F)
                bad |= np.abs(q - r) == F(0.5)
            pre = (np.cumsum(np.where(bad, F(0), r), dtype=F) + off).astype(F)   # exact: integers < 2^24
            cand = (s + np.ldexp(pre, k).astype(F)).astype(F)
            bad |= ~(cand < B)
            if not bad.any():
                off = pre[63]
                t += 64
                if t >= n:
                    s = cand[63]
                    break
                continue
            L = int(np.argmax(bad))
            sp = cand[L - 1] if L > 0 else F(s + F(np.ldexp(off, k)))
            s = F(sp + lanes[L])
            t += L + 1
            break
    return s


def test_model_equals_sequential_sum():
    for v in cases(seed=1, count=70, max_len=3000):
        a, b = sequential(v), model_sum(v)
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), (v.size, a, b)


def test_model_ties_and_binade_edges():
    # values landing exactly on half-ulp ties of a sum just below a power of two
    v = np.array([1.0, 0.5, 0.25] + [2.0 ** -24] * 40 + [3 * 2.0 ** -25] * 40 + [1.0 - 2.0 ** -24] * 30, F)
    assert sequential(v).view(np.uint32) == model_sum(v).view(np.uint32)
