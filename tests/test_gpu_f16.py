"""The F16 weight format on the device (WeightFormat::F16: matmul_f32,
weight_type.rs:228-270, on f16 weights; forward.rs with the F16Kernel):
the matmul and whole models against the oracle, bit for bit."""
import numpy as np
import pytest

from test_gpu_model import assert_bits

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("o,n,batch", [(300, 2048, 1), (64, 96, 1), (2048, 8192, 1), (130, 224, 7), (64, 64, 4),
                                       (3072, 2048, 1), (96, 160, 33)])
def test_matmul_f32_parity(gpu, oracle, o, n, batch):
    from yallma3_mini_inference_amd.weight_type import QuantizedWeight, matmul_f32
    rng = np.random.default_rng(o * 7 + n + batch)
    w16 = (rng.standard_normal((o, n)) * 0.05).astype(np.float16)
    x = rng.standard_normal((batch, n)).astype(np.float32)
    W = QuantizedWeight.upload_f16(w16, o, n)
    assert W.nbytes == o * n * 2
    got = matmul_f32(x, W, n, o)
    ref = np.zeros((batch, o), np.float32)
    oracle.matmul_f32(ref, x, w16.astype(np.float32), n, o)
    assert_bits(got, ref, "matmul_f32")


def test_matmul_f32_format_mismatch(gpu):
    import yallma3_mini_inference_amd as Y
    from yallma3_mini_inference_amd.weight_type import QuantizedWeight, WeightFormat, matmul_f32
    q = QuantizedWeight.upload(WeightFormat.Q8_0, np.ones(64 * 32, np.int8), np.ones(64, np.float32), 64, 32)
    with pytest.raises(Y.YlError, match="mismatch"):
        matmul_f32(np.ones((1, 32), np.float32), q, 32, 64)


def _pair(oracle, model_dir, name):
    from yallma3_mini_inference_amd import Transformer, synth
    path = synth.ensure(name, model_dir)
    return Transformer(path), oracle.Model(path)


@pytest.mark.parametrize("name,prompt_len,steps", [("tiny_f16", 20, 16), ("tiny_f16", 100, 4),
                                                    ("tiny_q8_f16emb", 20, 8), ("tiny_q8_f16emb", 90, 3),
                                                    ("small_f16", 70, 6)])
def test_f16_model_matches_oracle(gpu, oracle, model_dir, name, prompt_len, steps):
    g, o = _pair(oracle, model_dir, name)
    rng = np.random.default_rng(prompt_len + len(name))
    prompt = rng.integers(0, o.vocab, prompt_len).astype(np.uint32)
    gs, os_ = g.create_session(), o.create_session()
    assert_bits(g.forward_x(prompt, 0, gs), lo := o.forward_x(prompt, 0, os_), f"{name} prefill")
    tok, toks = oracle.argmax(lo), []
    first = tok
    for i in range(steps):
        lo = o.forward_x(np.array([tok], np.uint32), prompt_len + i, os_)
        assert_bits(g.forward_x(np.array([tok], np.uint32), prompt_len + i, gs), lo, f"{name} step {i}")
        tok = oracle.argmax(lo)
        toks.append(tok)
    # the device-chained greedy decode from a fresh session
    g2 = g.create_session()
    g.forward_x(prompt, 0, g2)
    assert list(g.generate_greedy(g2, first, prompt_len, steps)) == toks


def test_f16_kv_is_assigned(gpu, oracle, model_dir):
    """matmul_f32 assigns K and V (no `+=` as in the quantized path): running
    the same prompt twice without a reset gives the same logits."""
    g, o = _pair(oracle, model_dir, "tiny_f16")
    prompt = np.arange(1, 13, dtype=np.uint32)
    gs, os_ = g.create_session(), o.create_session()
    a = g.forward_x(prompt, 0, gs)
    b = g.forward_x(prompt, 0, gs)
    assert_bits(a, b, "rerun")
    o.forward_x(prompt, 0, os_)
    assert_bits(b, o.forward_x(prompt, 0, os_), "rerun vs oracle")
