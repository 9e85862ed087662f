"""Pins of the oracle's rope_gguf with YaRN scaling (util.rs:653-724) and of
the llama.attention.scale override (forward.rs:142-146) (CPU).

* Angle tables: the oracle's per-pair (cos, sin) under freq_scale != 1,
  ext_factor in {0.5, 1}, attn_factor != 1 and an original context shorter
  than the model's, against a float64 evaluation of the same formulas with the
  angle in closed form (tests/gguf_np.py yarn_cos_sin), within the f32 error
  bound attn * (theta_k * (k + 4) * 2^-23 + 4e-7) (the recurrence
  theta *= theta_scale loses about one ulp per pair).  Observed: <= 0.23 of
  the bound.  Four planted mistakes evaluated the same way -- the mix taken
  with freq_scale*theta in place of theta, corr_start without floor, no
  attn_factor, the ramp reversed -- each exceed the bound by more than 100x.
* Exact ends of the ramp: with ext_factor 1, pairs at or below corr_start
  take the unscaled angle, so their entries equal the default table's times
  attn_factor bit for bit; pairs at or past the upper correction dim take the
  interpolated angle, equal to the ext_factor-0 table's bit for bit.
* Composition: the float64 forward of tests/gguf_np.py, reading the
  llama.rope.scaling.* keys and llama.attention.scale from the GGUF, agrees
  with the oracle's logits to 1e-5 on YaRN models (observed <= 3.1e-7); the
  planted mistakes above and an ignored attention scale disagree by more than
  1e-4 (observed >= 2.4e-3).
"""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import gguf_np as G  # noqa: E402

# head size, rope base, scaling factor, ext_factor, attn_factor, original context
PARAMS = [
    (64, 10000.0, 4.0, 1.0, 1.1, 1024),
    (64, 500000.0, 8.0, 0.5, 0.9, 2048),
    (128, 500000.0, 32.0, 1.0, 1.0, 8192),
    (32, 500000.0, 4.0, 1.0, 1.2, 2048),
    (128, 10000.0, 2.0, 0.5, 1.05, 4096),
]
POSITIONS = [0, 1, 7, 100, 1000, 4095, 8191, 30000]


def _bound(pos, hd, base, attn):
    k = np.arange(hd // 2)
    theta = pos * float(base) ** (-2.0 * k / hd)
    return attn * (theta * (k + 4) * 2.0 ** -23 + 4e-7)


def _params(oracle, hd, base, f, e, a, n):
    return oracle.rope_params(hd, 1, 1, base, 1.0 / f, e, a, n)


def _corr_dims(hd, base, n):
    ln_b2 = 2.0 * np.log(base)
    low = max(np.floor(hd * np.log(n / (2 * np.pi * 32.0)) / ln_b2), 0.0)
    ce = hd * np.log(n / (2 * np.pi)) / ln_b2
    return low, min(low, ce) + min(ce, hd / 2) - low


@pytest.mark.parametrize("hd,base,f,e,a,n", PARAMS)
def test_yarn_table_within_float64_bound(oracle, hd, base, f, e, a, n):
    p = _params(oracle, hd, base, f, e, a, n)
    worst = 0.0
    for pos in POSITIONS:
        c, s = oracle.rope_cos_sin(p, pos)
        rc, rs = G.yarn_cos_sin(pos, hd, base, 1.0 / f, e, a, n)
        err = np.maximum(np.abs(c - rc), np.abs(s - rs)) / _bound(pos, hd, base, a)
        worst = max(worst, float(err.max()))
    assert worst <= 1.0, worst


@pytest.mark.parametrize("variant", G.YARN_VARIANTS)
@pytest.mark.parametrize("hd,base,f,e,a,n", PARAMS)
def test_yarn_planted_mistakes_exceed_the_bound(oracle, hd, base, f, e, a, n, variant):
    if variant == "yarn_no_attn_factor" and a == 1.0:
        pytest.skip("attn_factor 1: the mistake changes nothing")
    p = _params(oracle, hd, base, f, e, a, n)
    worst = 0.0
    for pos in POSITIONS[1:]:
        c, s = oracle.rope_cos_sin(p, pos)
        vc, vs = G.yarn_cos_sin(pos, hd, base, 1.0 / f, e, a, n, variant)
        worst = max(worst, float((np.maximum(np.abs(c - vc), np.abs(s - vs)) / _bound(pos, hd, base, a)).max()))
    assert worst > 100.0, worst


@pytest.mark.parametrize("hd,base,f,a,n", [(64, 10000.0, 4.0, 1.1, 1024), (32, 500000.0, 4.0, 1.2, 2048),
                                           (128, 500000.0, 32.0, 1.0, 8192)])
def test_yarn_ramp_ends_reduce_to_the_plain_tables(oracle, hd, base, f, a, n):
    low, high = _corr_dims(hd, base, n)
    k = np.arange(hd // 2)
    below, above = k <= low, k >= high
    assert below.any() and above.any()
    yarn = _params(oracle, hd, base, f, 1.0, a, n)
    plain = oracle.rope_params(hd, 1, 1, base, 1.0, 0.0, 1.0, n)
    interp = oracle.rope_params(hd, 1, 1, base, 1.0 / f, 0.0, a, n)
    for pos in POSITIONS:
        yc, ys = oracle.rope_cos_sin(yarn, pos)
        pc, ps = oracle.rope_cos_sin(plain, pos)
        ic, is_ = oracle.rope_cos_sin(interp, pos)
        # t = interp * 0 + theta * 1 = theta below the ramp
        np.testing.assert_array_equal(yc[below], pc[below] * np.float32(a))
        np.testing.assert_array_equal(ys[below], ps[below] * np.float32(a))
        # t = interp * 1 + theta * 0 = interp past it
        np.testing.assert_array_equal(yc[above], ic[above])
        np.testing.assert_array_equal(ys[above], is_[above])


def test_yarn_rotation_scales_pair_norms_by_attn_factor(oracle):
    rng = np.random.default_rng(3)
    hd, nh, nkv, a = 64, 4, 2, 1.1
    p = oracle.rope_params(hd, nh, nkv, 10000.0, 0.25, 1.0, a, 1024)
    q = rng.normal(0, 1, nh * hd).astype(np.float32)
    k = rng.normal(0, 1, nkv * hd).astype(np.float32)
    for pos in (0, 9, 3000):
        qq, kk = q.copy(), k.copy()
        oracle.rope_gguf(p, qq, kk, pos)
        for v, r in ((q, qq), (k, kk)):
            nv = np.hypot(v[0::2].astype(np.float64), v[1::2])
            nr = np.hypot(r[0::2].astype(np.float64), r[1::2])
            np.testing.assert_allclose(nr, a * nv, rtol=2e-6)


# --------------------------------------------------------------- composition

YARN_MODELS = {
    # name: (rope base, (factor, ext_factor, attn_factor, original ctx), attention.scale, FFN format)
    "yarn_q8": (10000.0, (4.0, 1.0, 1.1, 1024), 0.11, G.T_Q8_0),
    "yarn_q4_half": (500000.0, (8.0, 0.5, 0.9, 2048), 0.2, G.T_Q4_0),
}


def _yarn_model(tmp_path, name):
    base, sc, att, ffn = YARN_MODELS[name]
    return G.random_llama(str(tmp_path / f"{name}.gguf"), dim=128, n_heads=2, n_kv_heads=1, ctx=128,
                          ffn_fmt=ffn, seed=4, rope_theta=base, rope_scaling=sc, attention_scale=att)


def _compare(oracle, path, variant, prompt_len=40, steps=4):
    rng = np.random.default_rng(8)
    prompt = rng.integers(0, 96, prompt_len).astype(np.uint32)
    m = oracle.Model(path)
    s = m.create_session()
    f = G.Float64Model(G.Gguf(path), variant)
    lo = m.forward_x(prompt, 0, s)
    for t in prompt:
        lf = f.step(int(t))
    rel = lambda a, b: float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))
    worst = rel(lo, lf)
    tok = oracle.argmax(lo)
    for i in range(steps):
        lo = m.forward_x([tok], prompt_len + i, s)
        worst = max(worst, rel(lo, f.step(tok)))
        tok = oracle.argmax(lo)
    return worst


def test_oracle_reads_the_scaling_keys(oracle, tmp_path):
    path = _yarn_model(tmp_path, "yarn_q8")
    g = G.Gguf(path)
    assert g.meta["llama.rope.scaling.factor"] == np.float32(4.0)
    assert g.meta["llama.attention.scale"] == np.float32(0.11)
    # the same weights without the keys give different logits
    plain = G.random_llama(str(tmp_path / "plain.gguf"), dim=128, n_heads=2, n_kv_heads=1, ctx=128, seed=4)
    a, b = oracle.Model(path), oracle.Model(plain)
    la = a.forward_x(np.array([5, 9, 77], np.uint32), 0, a.create_session())
    lb = b.forward_x(np.array([5, 9, 77], np.uint32), 0, b.create_session())
    assert not np.array_equal(la, lb)


@pytest.mark.parametrize("name", sorted(YARN_MODELS))
def test_float64_forward_agrees_with_oracle_yarn(oracle, tmp_path, name):
    assert _compare(oracle, _yarn_model(tmp_path, name), "reference") < 1e-5


@pytest.mark.parametrize("variant", G.SCALING_VARIANTS)
@pytest.mark.parametrize("name", sorted(YARN_MODELS))
def test_oracle_rejects_yarn_and_scale_mistakes(oracle, tmp_path, name, variant):
    assert _compare(oracle, _yarn_model(tmp_path, name), variant) > 1e-4
