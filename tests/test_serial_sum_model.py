"""CPU model of the device's one-wavefront serial sum (wave_serial_sum_at in
csrc/yl_device.h), step by step in float32, held to the sequential f32 loop
it replaces.

While the running sum s stays in one binade it is a multiple of that binade's
ulp u, so a step adds v rounded to a multiple of u unless v/u is an exact
tie.  The first 32 values are added one at a time (the early sum crosses a
binade every few values).  Then super-rows of 64 lanes x KV values (lane l
holds KV consecutive values) are taken as integers r = rint(v/u): each lane
sums its own, a wavefront scan adds the lanes, and a super-row with no tie,
no value at or above the binade's top B and a last candidate below B is
taken whole.  Otherwise the first offending value in order gets one ordinary
f32 add onto the exact sum before it, and the same super-row is scanned
again from the next value with the new binade."""
import numpy as np

from serial_sum_cases import cases, sequential

F = np.float32
LANES = 64
PROLOGUE = 32


def _binade(s):
    ex = int(np.frexp(s)[1])
    k = max(ex - 24, -149)
    B = F(np.ldexp(1.0, ex)) if ex - 1 >= -126 else F(2.0 ** -126)
    return k, B


def _finish_nonfinite(s, v, start):
    # inf + finite = inf; a NaN anywhere after makes NaN
    if np.isnan(s) or np.isnan(v[start:]).any():
        return F(np.nan)
    return s


def model_sum(v, kv=8):
    v = np.asarray(v, F)
    n = v.size
    s = F(0.0)
    for i in range(min(n, PROLOGUE)):
        s = F(s + v[i])
    start = min(n, PROLOGUE)
    W = LANES * kv
    t0 = 0
    while start < n:
        if t0 + W <= start:
            t0 += W
            continue
        idx = t0 + np.arange(W)
        x = np.where(idx < n, v[np.minimum(idx, n - 1)], F(0)).astype(F).reshape(LANES, kv)
        idx = idx.reshape(LANES, kv)
        while start < min(n, t0 + W):
            if not np.isfinite(s):
                return _finish_nonfinite(s, v, start)
            live = idx >= start
            if s == 0:
                nz = np.nonzero((live & (x != 0)).ravel())[0]
                if nz.size == 0:
                    start = t0 + W
                    break
                s = x.ravel()[nz[0]]
                start = t0 + int(nz[0]) + 1
                continue
            k, B = _binade(s)
            with np.errstate(over="ignore", invalid="ignore"):   # only values already marked bad overflow
                q = np.ldexp(x, -k).astype(F)
                r = np.rint(q).astype(F)
                bad1 = live & (~(x < B) | (np.abs(q - r) == F(0.5)))
            rr = np.where(live & ~bad1, r, F(0)).astype(F)
            P = np.cumsum(rr, axis=1, dtype=F)             # in-lane prefix, exact integers
            T = P[:, -1]
            incl = np.cumsum(T, dtype=F)                    # wavefront scan of lane totals
            E = (incl - T).astype(F)
            cand_last = (s + np.ldexp(incl, k).astype(F)).astype(F)
            lane_bad = bad1.any(axis=1) | ~(cand_last < B)
            if not lane_bad.any():
                s = cand_last[-1]
                start = t0 + W
                break
            L = int(np.argmax(lane_bad))
            cand = (s + np.ldexp((E[L] + P[L]).astype(F), k).astype(F)).astype(F)
            badL = bad1[L] | (live[L] & ~(cand < B))
            i = int(np.argmax(badL))
            sp = cand[i - 1] if i > 0 else F(s + F(np.ldexp(E[L], k)))
            s = F(sp + x[L, i])
            start = t0 + L * kv + i + 1
        t0 += W
    if not np.isfinite(s):
        return _finish_nonfinite(s, v, n)
    return s


def _same(a, b):
    a, b = np.float32(a), np.float32(b)
    return (np.isnan(a) and np.isnan(b)) or a.view(np.uint32) == b.view(np.uint32)


def test_model_equals_sequential_sum():
    for kv in (8, 1):
        for v in cases(seed=1, count=70, max_len=3000):
            a, b = sequential(v), model_sum(v, kv)
            assert _same(a, b), (kv, v.size, a, b)


def test_model_ties_and_binade_edges():
    # values landing exactly on half-ulp ties of a sum just below a power of two
    v = np.array([1.0, 0.5, 0.25] + [2.0 ** -24] * 40 + [3 * 2.0 ** -25] * 40 + [1.0 - 2.0 ** -24] * 30 +
                 [2.0 ** -22] * 600, F)
    assert _same(sequential(v), model_sum(v))


def test_model_nonfinite():
    v = np.exp(-np.linspace(0, 4, 900)).astype(F)
    for bad in (np.inf, np.nan):
        w = v.copy()
        w[700] = bad
        assert _same(sequential(w), model_sum(w))
    w = v.copy()
    w[40] = np.inf
    w[800] = np.nan
    assert _same(sequential(w), model_sum(w))
