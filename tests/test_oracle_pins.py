"""Pins of the oracle's GGUF block decode and of its forward-pass composition
(CPU).

* Block decode (transformer_llama_gguf.rs:345-410, embedding dequant
  :453-489): GGUF files whose token embedding blocks are written by hand with
  known values -- Q8_0 int8 values, Q4_0 unsigned nibbles where byte j holds
  element 2j in its low nibble and 2j+1 in its high nibble, no offset -- and
  the oracle's dequantized table must equal value * scale element by element.
* Composition (forward.rs:120-280): an independent float64 forward over the
  same bytes (tests/gguf_np.py, its own GGUF parser) must agree with the
  oracle's logits to 1e-5 (relative, norm-wise; observed <= 3e-7, the
  activation quantization's rare rounding flips), on random models with
  distinct norm weights in Q8_0, Q4_0 and mixed formats; and each of a set of
  plausible mistakes -- GGML's Q4_0 nibble order and offset, HF-layout RoPE
  pairs, gate and up exchanged, the two norms exchanged, no 1/sqrt(head_size)
  scale -- computed the same way must disagree by more than 1e-4 (observed
  >= 1.1e-3).
* The golden fixture: the oracle's logits and greedy ids on seeded models,
  frozen in tests/golden/forward_golden.npz by tests/golden/make_golden.py,
  must be reproduced bit for bit.
"""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.join(HERE, "golden"))
import gguf_np as G  # noqa: E402


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def _hand_embedding_model(path, fmt):
    """Model whose token_embd blocks are hand-written: row v, element e holds
    value (7e + 3v) mod 16 (Q4_0, unsigned) or ((7e + 3v) mod 255) - 127
    (Q8_0), block scale 2^-(b + 1) * (1 + v/64)."""
    dim, vocab = 64, 96
    e = np.arange(dim)[None, :]
    v = np.arange(vocab)[:, None]
    nb = dim // 32
    d = (2.0 ** -(np.arange(nb)[None, :] + 1) * (1 + v / 64.0)).astype(np.float16)
    if fmt == G.T_Q4_0:
        vals = (7 * e + 3 * v) % 16
        blob = G.q4_blocks(vals.ravel(), d.ravel())
    else:
        vals = (7 * e + 3 * v) % 255 - 127
        blob = G.q8_blocks(vals.ravel(), d.ravel())
    G.random_llama(path, dim=dim, vocab=vocab, n_heads=2, n_kv_heads=1, seed=5)   # head size 32
    g = G.Gguf(path)
    tensors = []
    for name, (dims, typ, off) in g.tensors.items():
        raw, _ = g.raw(name)
        if name == "token_embd.weight":
            tensors.append((name, dims, fmt, blob))
        else:
            tensors.append((name, dims, typ, raw.tobytes()))
    meta = [(k, g.meta_type[k], (G._STR, g.meta[k]) if g.meta_type[k] == G._ARR else g.meta[k]) for k in g.meta]
    G.write(path, meta, tensors)
    expect = vals.astype(np.float64) * np.repeat(d.astype(np.float64), 32, axis=1)
    return expect


@pytest.mark.parametrize("fmt", [G.T_Q8_0, G.T_Q4_0])
def test_oracle_decodes_hand_built_blocks(oracle, tmp_path, fmt):
    path = str(tmp_path / f"hand_{fmt}.gguf")
    expect = _hand_embedding_model(path, fmt)
    m = oracle.Model(path)
    got = m.embedding().reshape(m.vocab, m.dim).astype(np.float64)
    np.testing.assert_array_equal(got, expect)
    # the numpy reader decodes the same bytes to the same values
    np.testing.assert_array_equal(G.Gguf(path).f32("token_embd.weight").reshape(m.vocab, m.dim), expect)


def test_q4_ggml_order_differs_from_the_reference_order(tmp_path):
    # the negative control used below is a real difference on these bytes
    path = str(tmp_path / "hand_q4.gguf")
    expect = _hand_embedding_model(path, G.T_Q4_0)
    q, d = G.Gguf(path).quantized("token_embd.weight", "ggml")
    assert not np.array_equal(q.astype(np.float64) * np.repeat(d, 32), expect.ravel())


MODELS = {  # attention, FFN, embedding formats
    "q8": (G.T_Q8_0, G.T_Q8_0, G.T_Q8_0),
    "q4": (G.T_Q4_0, G.T_Q4_0, G.T_Q4_0),
    "mixed_ffn_q4": (G.T_Q8_0, G.T_Q4_0, G.T_Q8_0),
    "embd_q4": (G.T_Q8_0, G.T_Q8_0, G.T_Q4_0),
}
PROMPT = [3, 17, 55, 2, 90, 41]


def _compare(oracle, path, variant, steps=4):
    m = oracle.Model(path)
    s = m.create_session()
    f = G.Float64Model(G.Gguf(path), variant)
    lo = m.forward_x(np.array(PROMPT, np.uint32), 0, s)
    for t in PROMPT:
        lf = f.step(t)
    worst = _rel(lo, lf)
    tok = oracle.argmax(lo)
    for i in range(steps):
        lo = m.forward_x([tok], len(PROMPT) + i, s)
        worst = max(worst, _rel(lo, f.step(tok)))
        tok = oracle.argmax(lo)
    return worst


@pytest.mark.parametrize("name", sorted(MODELS))
def test_float64_forward_agrees_with_oracle(oracle, tmp_path, name):
    a, f, e = MODELS[name]
    path = G.random_llama(str(tmp_path / f"{name}.gguf"), attn_fmt=a, ffn_fmt=f, embd_fmt=e, seed=1)
    assert _compare(oracle, path, "reference") < 1e-5


@pytest.mark.parametrize("variant", G.BASE_VARIANTS)
@pytest.mark.parametrize("name", ["mixed_ffn_q4", "embd_q4"])
def test_oracle_rejects_plausible_mistakes(oracle, tmp_path, name, variant):
    a, f, e = MODELS[name]
    path = G.random_llama(str(tmp_path / f"{name}.gguf"), attn_fmt=a, ffn_fmt=f, embd_fmt=e, seed=1)
    assert _compare(oracle, path, variant) > 1e-4


def test_golden_fixture_reproduced(oracle, tmp_path):
    import make_golden
    ref = np.load(make_golden.FIXTURE)
    got = make_golden.compute(oracle, str(tmp_path))
    assert sorted(ref.files) == sorted(got)
    for k in ref.files:
        a, b = np.asarray(ref[k]), np.asarray(got[k])
        assert a.dtype == b.dtype and a.shape == b.shape, k
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), k
