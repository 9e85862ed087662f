"""Pins the CPU oracle (oracle/yl_oracle.c) without re-typing its formulas.

Each check comes from somewhere other than the oracle's own code: the
reference's known-answer test, IEEE/numpy for exact primitives, closed forms
with exactly representable values, float64 textbook math within tolerance,
or invariants (rotation preserves norms, one key -> output = value) chosen so
a plausible slip (wrong qmax, banker's rounding, swapped scale, missing
`+=`, half-split instead of consecutive RoPE pairs, wrong mask) fails.
"""
import numpy as np
import pytest


def test_matmul_reference_kat(oracle):
    # tests/matmul_q8_tests.rs:30-53: n=64, o=33 (tail column path), all ones -> n
    n, o = 64, 33
    out = np.zeros(o, np.float32)
    oracle.matmul_q8_slices(out, np.ones(n, np.int8), np.ones(2, np.float32), np.ones(o * n, np.int8),
                            np.ones(o * n // 32, np.float32), n, o)
    assert np.all(np.abs(out - n) < 1e-5)


def test_matmul_f32_pins(oracle):
    """weight_type.rs:228-270: every column assigned (no `+=`); sums of exactly
    representable terms are exact; the column order of the f32 chain matters
    (1 + 2^-24 ... does not round the same as the reversed order)."""
    n, o = 64, 5
    out = np.full(o, 7.0, np.float32)
    oracle.matmul_f32(out, np.ones(n, np.float32), np.full(o * n, 0.5, np.float32), n, o)
    assert np.all(out == 32.0)                        # assigned, not accumulated
    # order-sensitive chain: x = [1, 2^-24 x 63]: left to right each tiny term
    # rounds away (ties to even), so the sum stays 1
    x = np.array([1.0] + [2.0 ** -24] * 63, np.float32)
    out = np.zeros(1, np.float32)
    oracle.matmul_f32(out, x, np.ones(64, np.float32), 64, 1)
    assert out[0] == 1.0
    out2 = np.zeros(1, np.float32)
    oracle.matmul_f32(out2, x[::-1].copy(), np.ones(64, np.float32), 64, 1)
    assert out2[0] > 1.0                              # the reversed order keeps them
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 96)).astype(np.float32)
    w = rng.standard_normal((7, 96)).astype(np.float16).astype(np.float32)
    out = np.zeros((3, 7), np.float32)
    oracle.matmul_f32(out, x, w, 96, 7)
    np.testing.assert_allclose(out, x.astype(np.float64) @ w.astype(np.float64).T, rtol=1e-5, atol=1e-5)


def test_f16_all_patterns(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    mine = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    same = (mine.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(mine) & np.isnan(ref))
    assert same.all()


def test_expf_correctly_rounded(oracle):
    rng = np.random.default_rng(1)
    xs = np.concatenate([rng.uniform(-104, 88.7, 60000), rng.uniform(-10, 10, 60000),
                         np.array([0.0, -0.0, 1.0, -1.0, 88.72, -87.3, -103.9])]).astype(np.float32)
    mine = np.array([oracle.expf(float(x)) for x in xs], np.float32)
    with np.errstate(over="ignore"):
        ref = np.exp(xs.astype(np.float64)).astype(np.float32)
    assert (mine.view(np.uint32) == ref.view(np.uint32)).all()
    assert oracle.expf(-1e10) == 0.0 and oracle.expf(100.0) == np.inf


def test_quantize_q8_properties(oracle):
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, 32 * 64).astype(np.float32)
    x[32:64] = 0.0                                    # all-zero group
    q, s = oracle.quantize(oracle.Q8_0, x)
    g = x.reshape(-1, 32)
    assert s[1] == 0.0 and (q[32:64] == 0).all()      # 0/0 -> NaN -> 0 (saturating cast)
    amax = np.abs(g).max(axis=1)
    np.testing.assert_array_equal(s, (amax / np.float32(127.0)).astype(np.float32))
    qi = q.reshape(-1, 32).astype(np.int32)
    live = s > 0
    # the element equal to absmax maps to +-127
    arg = np.abs(g).argmax(axis=1)
    assert (np.abs(qi[np.arange(len(qi)), arg])[live] == 127).all()
    # dequantization error within half a step
    err = np.abs(g - qi * s[:, None])
    assert (err[live] <= s[live, None] * 0.5000001).all()


def test_quantize_rounds_half_away_from_zero(oracle):
    # scale = 127/127 = 1 exactly; x/1 = k + 0.5 must round away from zero (Rust f32::round)
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:7] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5]
    q, s = oracle.quantize(oracle.Q8_0, x)
    assert s[0] == 1.0
    assert list(q[:7]) == [127, 1, 2, 3, -1, -2, -3]


def test_quantize_q4_properties(oracle):
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, 32 * 50).astype(np.float32)
    q, s = oracle.quantize(oracle.Q4_0, x)
    g = x.reshape(-1, 32)
    np.testing.assert_array_equal(s, (np.abs(g).max(axis=1) / np.float32(7.0)).astype(np.float32))
    assert q.min() >= -7 and q.max() <= 7
    qi = q.reshape(-1, 32)
    arg = np.abs(g).argmax(axis=1)
    assert (np.abs(qi[np.arange(len(qi)), arg]) == 7).all()
    assert (np.abs(g - qi * s[:, None]) <= s[:, None] * 0.5000001).all()


def _pow2_case(rng, batch, n, o):
    # |isum| <= 32*7*7 < 2^11 and scales 2^-3 * {2^-6, 2^-7}: each term is a
    # multiple of 2^-10 below 2^2, so every partial sum fits a binary32 exactly
    x = rng.integers(-7, 8, batch * n).astype(np.int8)
    w = rng.integers(-7, 8, o * n).astype(np.int8)
    xs = np.full(batch * n // 32, 2.0 ** -3, np.float32)
    ws = (2.0 ** rng.integers(-7, -5, o * n // 32)).astype(np.float32)
    return x, xs, w, ws


def test_matmul_exact_closed_form(oracle):
    # Power-of-two scales make every block term exact, and the partial sums
    # stay exactly representable (few blocks, bounded magnitudes) -- so the
    # result must equal the float64 sum of int64 block dots exactly.
    rng = np.random.default_rng(4)
    batch, n, o = 3, 96, 10
    x, xs, w, ws = _pow2_case(rng, batch, n, o)
    init = np.round(rng.normal(0, 4, batch * o)).astype(np.float32) * np.float32(0.25)
    out = init.copy()
    oracle.matmul_q8_slices(out, x, xs, w, ws, n, o)
    xb = x.astype(np.int64).reshape(batch, n // 32, 32)
    wb = w.astype(np.int64).reshape(o, n // 32, 32)
    dots = np.einsum("rbk,cbk->rcb", xb, wb).astype(np.float64)
    terms = dots * ws.reshape(o, n // 32)[None] * xs.reshape(batch, n // 32)[:, None]
    expect = terms.sum(axis=2)
    acc_cols = (o // 4) * 4                                # `+=` columns keep the old value
    expect[:, :acc_cols] += init.reshape(batch, o)[:, :acc_cols]
    np.testing.assert_array_equal(out.reshape(batch, o), expect.astype(np.float32))


def test_matmul_float64_bound(oracle):
    rng = np.random.default_rng(5)
    n, o = 512, 64
    xf = rng.normal(0, 1, n).astype(np.float32)
    wf = rng.normal(0, 0.02, o * n).astype(np.float32)
    xq, xs = oracle.quantize(oracle.Q8_0, xf)
    wq, ws = oracle.quantize(oracle.Q8_0, wf)
    out = np.zeros(o, np.float32)
    oracle.matmul_q8_slices(out, xq, xs, wq, ws, n, o)
    deq_x = xq.astype(np.float64) * np.repeat(xs, 32)
    deq_w = wq.astype(np.float64).reshape(o, n) * np.repeat(ws, 32).reshape(o, n)
    ref = deq_w @ deq_x
    assert np.max(np.abs(out - ref)) <= 1e-5 * np.max(np.abs(ref)) + 1e-6


def test_rmsnorm_textbook_and_tail(oracle):
    rng = np.random.default_rng(6)
    x = rng.normal(0, 3, 2048).astype(np.float32)
    w = rng.normal(1, 0.1, 2048).astype(np.float32)
    o = oracle.rmsnorm(x, w, 1e-5)
    x64 = x.astype(np.float64)
    ref = w * x64 / np.sqrt(np.mean(x64 ** 2) + 1e-5)
    np.testing.assert_allclose(o, ref, rtol=2e-6, atol=1e-7)
    # size % 8 tail: only the first 8 elements are summed and written (util.rs:397-425)
    x13 = rng.normal(0, 1, 13).astype(np.float32)
    o13 = oracle.rmsnorm(x13, np.ones(13, np.float32), 1e-5)
    ss = np.sum(x13[:8].astype(np.float64) ** 2) / 13
    np.testing.assert_allclose(o13[:8], x13[:8] / np.sqrt(ss + 1e-5), rtol=2e-6)
    assert (o13[8:] == 0).all()


def test_rope_identity_norms_and_pairing(oracle):
    rng = np.random.default_rng(7)
    p = oracle.rope_params(64, 4, 2, 10000.0)
    q = rng.normal(0, 1, 256).astype(np.float32)
    k = rng.normal(0, 1, 128).astype(np.float32)
    q0, k0 = q.copy(), k.copy()
    oracle.rope_gguf(p, q0, k0, 0)
    np.testing.assert_array_equal(q0, q)
    np.testing.assert_array_equal(k0, k)
    for pos in (1, 7, 10):
        qq, kk = q.copy(), k.copy()
        oracle.rope_gguf(p, qq, kk, pos)
        # textbook consecutive-pair rotation with angle pos * theta^(-2i/hd)
        i = np.arange(32)
        ang = pos * 10000.0 ** (-2.0 * i / 64)
        c, s = np.cos(ang), np.sin(ang)
        for vec, rot in ((q, qq), (k, kk)):
            v = vec.astype(np.float64).reshape(-1, 32, 2)
            ref = np.stack([v[..., 0] * c - v[..., 1] * s, v[..., 0] * s + v[..., 1] * c], -1).ravel()
            np.testing.assert_allclose(rot, ref, rtol=0, atol=2e-4)
            nr = np.hypot(rot.reshape(-1, 2)[:, 0], rot.reshape(-1, 2)[:, 1])
            nv = np.hypot(vec.reshape(-1, 2)[:, 0], vec.reshape(-1, 2)[:, 1])
            np.testing.assert_allclose(nr, nv, rtol=1e-5)


def _attention64(q, kc, vc, batch, start, nh, nkv, hd, scale):
    seq = start + batch
    out = np.zeros((batch, nh, hd))
    K = kc.reshape(-1, nkv, hd)[:seq].astype(np.float64)
    V = vc.reshape(-1, nkv, hd)[:seq].astype(np.float64)
    Q = q.reshape(batch, nh, hd).astype(np.float64)
    for t in range(batch):
        for h in range(nh):
            kvh = h // (nh // nkv)
            sc = K[: start + t + 1, kvh] @ Q[t, h] * scale
            p = np.exp(sc - sc.max())
            p /= p.sum()
            out[t, h] = p @ V[: start + t + 1, kvh]
    return out.ravel()


def test_attention_brute_force(oracle):
    rng = np.random.default_rng(8)
    nh, nkv, hd = 4, 2, 64
    for batch, start in ((1, 0), (1, 37), (5, 11), (9, 0)):
        seq = start + batch
        q = rng.normal(0, 1, batch * nh * hd).astype(np.float32)
        kc = rng.normal(0, 1, seq * nkv * hd).astype(np.float32)
        vc = rng.normal(0, 1, seq * nkv * hd).astype(np.float32)
        out = oracle.fused_attention(q, kc, vc, seq, batch, nh, nkv, hd, start, nkv * hd, 0.125)
        ref = _attention64(q, kc, vc, batch, start, nh, nkv, hd, 0.125)
        np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)


def test_attention_single_key_returns_value(oracle):
    rng = np.random.default_rng(9)
    q = rng.normal(0, 1, 2 * 32).astype(np.float32)
    kc = rng.normal(0, 1, 32).astype(np.float32)
    vc = rng.normal(0, 1, 32).astype(np.float32)
    out = oracle.fused_attention(q, kc, vc, 1, 1, 2, 1, 32, 0, 32, 0.3)
    np.testing.assert_array_equal(out, np.concatenate([vc, vc]))


def test_swiglu_closed_form(oracle):
    rng = np.random.default_rng(10)
    g = rng.normal(0, 2, 1000).astype(np.float32)
    u = rng.normal(0, 1, 1000).astype(np.float32)
    h = oracle.swiglu(g, u)
    g64 = g.astype(np.float64)
    np.testing.assert_allclose(h, g64 / (1 + np.exp(-g64)) * u, rtol=3e-7, atol=1e-8)


def test_logits_and_argmax(oracle):
    rng = np.random.default_rng(11)
    dim, vocab = 96, 300
    last = rng.normal(0, 1, dim).astype(np.float32)
    emb = rng.normal(0, 0.02, vocab * dim).astype(np.float32)
    lg = oracle.logits(last, emb, vocab, dim)
    np.testing.assert_allclose(lg, emb.reshape(vocab, dim).astype(np.float64) @ last, rtol=1e-5, atol=1e-6)
    assert oracle.argmax(np.array([1.0, 3.0, 3.0, -1.0], np.float32)) == 1   # first maximum
    assert oracle.argmax(np.array([-2.0, -2.0], np.float32)) == 0
