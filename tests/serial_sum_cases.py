"""Adversarial inputs for the serial f32 sum ((0 + v0) + v1) + ... of
nonnegative values: softmax-like exponentials, underflowing and subnormal
values, zeros, dyadic values with exact rounding ties, a subnormal start, and
rare large jumps across several binades."""
import numpy as np


def cases(seed=0, count=120, max_len=9000):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        n = int(rng.integers(1, max_len)) if i % 4 else int(rng.integers(1, 200))
        kind = i % 7
        if kind == 0:
            v = np.exp(-rng.uniform(0, 1 + 30 * rng.random(), n))
        elif kind == 1:
            v = np.exp(-rng.uniform(0, 110, n))
        elif kind == 2:
            v = np.where(rng.random(n) < 0.25, 0.0, np.exp(-rng.uniform(0, 8, n)))
        elif kind == 3:
            v = np.ldexp(rng.integers(0, 64, n).astype(np.float64), -rng.integers(0, 12, n))
        elif kind == 4:
            v = np.exp(-rng.uniform(0, 3, n))
            v[0] = 1e-40
        elif kind == 5:
            v = np.where(rng.random(n) < 0.01, 1.0, rng.random(n) * 1e-6)
        else:
            v = rng.integers(0, 3, n) * 0.5 + np.ldexp(1.0, -rng.integers(0, 30, n))
        out.append(v.astype(np.float32))
    out.append(np.zeros(0, np.float32))
    out.append(np.zeros(130, np.float32))
    return out


def sequential(v):
    """The one-at-a-time f32 loop (numpy's accumulate adds sequentially)."""
    v = np.asarray(v, np.float32)
    return np.float32(0.0) if v.size == 0 else np.cumsum(v, dtype=np.float32)[-1]
