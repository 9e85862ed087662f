"""The HIP path against hand-built inputs and the frozen golden fixture,
without the oracle in between.

* GGUF block decode on the device (transformer_llama_gguf.rs:345-410): hand-
  written Q8_0 / Q4_0 blocks uploaded with yl_weight_upload_gguf, multiplied
  by one-hot activations, must return value * scale for every element (the
  Q4_0 nibble order lo -> 2j, hi -> 2j+1, no offset); the same blocks as a
  model's token embedding must dequantize to value * scale.
* Greedy argmax on NaN logits (sampler.rs:67-79 starts from row 0 and
  replaces the maximum only on `p > max`): a NaN in row 0 returns 0, a NaN
  elsewhere never wins, all-NaN logits return 0.
* tests/golden/forward_golden.npz: prefill logits, greedy ids and last-step
  logits of three seeded models, bit for bit.
"""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.join(HERE, "golden"))
import gguf_np as G  # noqa: E402


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("batch", [64, 1])
def test_weight_blocks_decode_by_hand(gpu, fmt, batch):
    """Row r, element e holds (5e + 11r) mod 16 (Q4_0) or ((5e + 11r) mod 255)
    - 127 (Q8_0), block scale 2^-(b+2) * (1 + r/32).  Activation row k is the
    one-hot e_k, quantized to q = qmax at k with scale 1/qmax; the matmul
    then returns ((float)(qmax * value) * scale) * (1/qmax)."""
    from yallma3_mini_inference_amd import QuantizedWeight, WeightFormat, matmul
    o, n = 40, 64
    r = np.arange(o)[:, None]
    e = np.arange(n)[None, :]
    d = (2.0 ** -(np.arange(n // 32)[None, :] + 2) * (1 + r / 32.0)).astype(np.float16)
    if fmt == 1:
        vals, qmax = (5 * e + 11 * r) % 16, 7
        blob = G.q4_blocks(vals.ravel(), d.ravel())
    else:
        vals, qmax = (5 * e + 11 * r) % 255 - 127, 127
        blob = G.q8_blocks(vals.ravel(), d.ravel())
    w = QuantizedWeight.upload_gguf(WeightFormat(fmt), blob, o, n)
    ks = np.arange(n) if batch > 1 else np.array([37])
    xq = np.zeros((ks.size, n), np.int8)
    xq[np.arange(ks.size), ks] = qmax
    xs = np.full((ks.size, n // 32), np.float32(1.0) / np.float32(qmax), np.float32)
    out = matmul(np.zeros(ks.size * o, np.float32), xq.ravel(), xs.ravel(), w, n, o).reshape(ks.size, o)
    dk = d.astype(np.float32)[:, ks // 32].T                        # [k][r]
    expect = (vals[:, ks].T * qmax).astype(np.float32) * dk * xs[:, :1]
    assert np.array_equal(_bits(out), _bits(expect))


@pytest.mark.parametrize("fmt", [G.T_Q8_0, G.T_Q4_0])
def test_embedding_blocks_decode_by_hand(gpu, tmp_path, fmt):
    from test_oracle_pins import _hand_embedding_model
    from yallma3_mini_inference_amd import Transformer
    path = str(tmp_path / f"hand_{fmt}.gguf")
    expect = _hand_embedding_model(path, fmt)
    t = Transformer(path)
    got = t.get_embeddings_batch(np.arange(expect.shape[0], dtype=np.uint32))
    assert np.array_equal(got.astype(np.float64), expect)


@pytest.mark.parametrize("case", ["row0", "row7", "all"])
def test_greedy_argmax_on_nan_logits(gpu, oracle, tmp_path, case):
    from yallma3_mini_inference_amd import Transformer
    kw = {"row0": {"nan_embedding_rows": (0,)}, "row7": {"nan_embedding_rows": (7,)},
          "all": {"nan_output_norm": True}}[case]
    path = G.random_llama(str(tmp_path / f"nan_{case}.gguf"), seed=3, emb_std=0.05, w_std=0.2, **kw)
    g, o = Transformer(path), oracle.Model(path)
    prompt = np.array([5, 9, 13, 21], np.uint32)
    gs, os_ = g.create_session(), o.create_session()
    lg, lo = g.forward_x(prompt, 0, gs), o.forward_x(prompt, 0, os_)
    nan = np.isnan(lo)
    assert np.array_equal(np.isnan(lg), nan)
    assert np.array_equal(_bits(lg)[~nan], _bits(lo)[~nan])
    want = oracle.argmax(lo)
    if case == "row0":
        assert nan[0] and want == 0
    elif case == "row7":
        assert nan[7] and not nan[0] and want != 7
    else:
        assert nan.all() and want == 0
    gs2 = g.create_session()
    assert g.forward_argmax(prompt, 0, gs2) == want
    ref, tok = [], want
    for i in range(3):
        tok = oracle.argmax(o.forward_x([tok], len(prompt) + i, os_))
        ref.append(tok)
    assert list(g.generate_greedy(gs2, want, len(prompt), 3)) == ref


def test_golden_fixture_on_device(gpu, tmp_path):
    import make_golden
    from yallma3_mini_inference_amd import Transformer
    ref = np.load(make_golden.FIXTURE)
    for name in make_golden.MODELS:
        t = Transformer(make_golden.model_path(name, str(tmp_path)))
        p = ref[f"{name}_prompt"]
        s, s2 = t.create_session(), t.create_session()
        lg = t.forward_x(p, 0, s)
        assert np.array_equal(_bits(lg), _bits(ref[f"{name}_prefill_logits"])), name
        first = int(np.argmax(lg))
        ids = ref[f"{name}_greedy"]
        tok = first
        for i in range(make_golden.STEPS):
            lg = t.forward_x([tok], len(p) + i, s)
            tok = int(ids[i])
        assert np.array_equal(_bits(lg), _bits(ref[f"{name}_last_logits"])), name
        t.forward_argmax(p, 0, s2)
        assert list(t.generate_greedy(s2, first, len(p), make_golden.STEPS)) == list(ids), name
