"""Parity at the benchmark configurations' full model shapes.

Each test builds the seeded synthetic GGUF of a benchmark configuration
(weights ~N(0, 0.02), GGUF Q8_0/Q4_0 blocks) and runs the HIP path and the
oracle on the same inputs:

  SmolLM2-135M Q8_0      256 random prompt ids, then 128 greedy tokens
  Llama-3.2-1B Q8_0      512 random prompt ids, then 256 greedy tokens
  Llama-3.2-1B Q4_0      512- and 2048-token prompts (int8-MFMA GEMM and the
                         tiled prompt attention), then greedy steps
  Llama-3-8B mixed       Q4_0 FFN + Q8_0 attention/output, KV cache random-
                         filled to 8192 positions (the oracle cannot prefill
                         8192 tokens of this shape in test time), then
                         teacher-forced and greedy decode steps

Bar (forward.rs:120-297, sampler.rs:67-79): logits bit-identical to the
oracle's at every compared step -- which implies the 1e-3 relative bar the
north star states, and the largest relative difference is reported -- and
identical greedy token ids.  Prompt ids are uniform over the vocabulary
(seeded), as the configurations specify.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3   # the stated tolerance; bit-exactness is asserted on top of it


def rel_diff(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def assert_logits(lg, lo, what):
    r = rel_diff(lg, lo)
    assert r <= REL_TOL, f"{what}: max relative difference {r:.3g} above {REL_TOL}"
    a = np.ascontiguousarray(lg, np.float32).view(np.uint32)
    b = np.ascontiguousarray(lo, np.float32).view(np.uint32)
    bad = np.nonzero(a != b)[0]
    assert bad.size == 0, f"{what}: {bad.size} logits differ in their bits (max rel {r:.3g}), first {bad[:4]}"
    return r


def _models(oracle, model_dir, name):
    from yallma3_mini_inference_amd import Transformer, synth
    path = synth.ensure(name, model_dir)
    return Transformer(path), oracle.Model(path)


def _prompt_then_greedy(oracle, g, o, n_prompt, n_steps, seed, compare_steps):
    """Prefill a random prompt on both, then n_steps greedy tokens: the
    device's chained generate_greedy against the oracle's own greedy chain,
    and the logits of the first compare_steps steps through forward_x."""
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, o.vocab, n_prompt).astype(np.uint32)
    gs, gs2, os_ = g.create_session(), g.create_session(), o.create_session()
    lo = o.forward_x(prompt, 0, os_)
    worst = assert_logits(g.forward_x(prompt, 0, gs), lo, f"{n_prompt}-token prefill")
    first = oracle.argmax(lo)
    assert g.forward_argmax(prompt, 0, gs2) == first
    ref, tok = [], first
    for i in range(n_steps):
        pos = n_prompt + i
        lo = o.forward_x([tok], pos, os_)
        if i < compare_steps:
            worst = max(worst, assert_logits(g.forward_x([tok], pos, gs), lo, f"step {i} (position {pos})"))
        tok = oracle.argmax(lo)
        ref.append(tok)
    got = g.generate_greedy(gs2, first, n_prompt, n_steps)
    assert list(got) == ref, f"greedy tokens differ from step {int(np.argmax(np.asarray(got) != ref))}"
    print(f"max relative logit difference {worst:.3g} over {compare_steps + 1} compared passes")
    return gs, os_


def test_smollm2_135m_q8_full_config(gpu, oracle, model_dir):
    g, o = _models(oracle, model_dir, "smollm2_135m")
    _prompt_then_greedy(oracle, g, o, 256, 128, seed=135, compare_steps=128)


@pytest.mark.timeout(600)
def test_llama32_1b_q8_full_config(gpu, oracle, model_dir):
    """The headline workload: 512 prompt ids then 256 greedy tokens, KV f32
    at ctx 4096.  Every decode step's logits are compared (the step is the
    fused decode graph: QKV+RoPE, attention, Wo, gate/up+SwiGLU, down, logits
    over the 128256 x 2048 table)."""
    g, o = _models(oracle, model_dir, "llama32_1b")
    assert g.max_ctx_len() == 4096
    gs, os_ = _prompt_then_greedy(oracle, g, o, 512, 256, seed=512, compare_steps=256)
    n = 512 + 256
    np.testing.assert_array_equal(gs.key_cache()[:, :n].view(np.uint32), os_.key_cache()[:, :n].view(np.uint32))
    np.testing.assert_array_equal(gs.value_cache()[:, :n].view(np.uint32),
                                  os_.value_cache()[:, :n].view(np.uint32))


@pytest.mark.timeout(600)
@pytest.mark.parametrize("n_prompt,n_steps", [(512, 8), (2048, 2)])
def test_llama32_1b_q4_prefill(gpu, oracle, model_dir, n_prompt, n_steps):
    """Q4_0 weights and activations (reference semantics, weight_type.rs:52-74
    and transformer_llama_gguf.rs:375-410): the prompt's projections run on the
    int8-MFMA GEMM and its attention on the tiled prompt kernels; then greedy
    decode steps on the Q4_0 GEMVs."""
    g, o = _models(oracle, model_dir, "llama32_1b_q4")
    _prompt_then_greedy(oracle, g, o, n_prompt, n_steps, seed=n_prompt, compare_steps=n_steps)


@pytest.mark.timeout(900)
def test_llama3_8b_mixed_decode_at_8k(gpu, oracle, model_dir):
    """dim 4096, FFN 14336 (Q4_0), attention/output Q8_0, 32 layers, head size
    128, 4 query heads per kv head, ctx 8448.  The KV cache below 8192 is the
    same random fill on both sides; decode at 8192.. runs the split attention
    (scores, softmax, P.V by lane, output) in the decode graph, the 16-lane
    QKV GEMV with its RoPE epilogue, and the Q4_0 gate/up and down GEMVs."""
    g, o = _models(oracle, model_dir, "llama3_8b_mixed")
    P = 8192
    rng = np.random.default_rng(8192)
    gs, gs2, os_ = g.create_session(), g.create_session(), o.create_session()
    k = rng.standard_normal((o.n_layers, P, o.kv_dim), dtype=np.float32)
    v = rng.standard_normal((o.n_layers, P, o.kv_dim), dtype=np.float32)
    os_.key_cache()[:, :P] = k
    os_.value_cache()[:, :P] = v
    gs.upload_kv(k, v)
    gs2.upload_kv(k, v)
    del k, v
    tok, ref, worst = 128000, [], 0.0
    for pos in range(P, P + 3):
        lo = o.forward_x([tok], pos, os_)
        worst = max(worst, assert_logits(g.forward_x([tok], pos, gs), lo, f"decode at {pos}"))
        tok = oracle.argmax(lo)
        ref.append(tok)
    assert list(g.generate_greedy(gs2, 128000, P, 3)) == ref
    print(f"max relative logit difference {worst:.3g}")


@pytest.mark.timeout(600)
def test_llama3_8b_layer_shape_prefill_chunk_at_7680(gpu, oracle, model_dir):
    """The Llama-3-8B configuration's prefill leg at its own layer shape: a
    256-token prompt chunk at positions 7680..7935 over a random KV cache
    below 7680 (the same on both sides), then two decode steps.  The chunk's
    projections run on the int8-MFMA GEMM at K = 4096 and, for the Q4_0 down
    projection, K = 14336 (448 blocks per row); its attention runs the tiled
    prompt kernels at head size 128 over 7,936 positions; the logits cover
    the 128,256-row table.  The model has two layers of the 8B shape (dim
    4096, FFN 14336 Q4_0, attention Q8_0, 32/8 heads): every launch is the
    32-layer model's, which repeats them, and the oracle finishes two layers
    of this chunk in test time (forward.rs:120-280)."""
    g, o = _models(oracle, model_dir, "llama3_8b_mixed_2l")
    P, B = 7680, 256
    rng = np.random.default_rng(7680)
    k = rng.standard_normal((o.n_layers, P, o.kv_dim), dtype=np.float32)
    v = rng.standard_normal((o.n_layers, P, o.kv_dim), dtype=np.float32)
    gs, os_ = g.create_session(), o.create_session()
    os_.key_cache()[:, :P] = k
    os_.value_cache()[:, :P] = v
    gs.upload_kv(k, v)
    del k, v
    prompt = rng.integers(0, o.vocab, B).astype(np.uint32)
    lo = o.forward_x(prompt, P, os_)
    worst = assert_logits(g.forward_x(prompt, P, gs), lo, f"{B}-token chunk at {P}")
    kc, vc = gs.key_cache(), gs.value_cache()
    ok, ov = os_.key_cache(), os_.value_cache()
    for l in range(o.n_layers):
        assert np.array_equal(kc[l, P:P + B].view(np.uint32), ok[l, P:P + B].view(np.uint32)), f"K layer {l}"
        assert np.array_equal(vc[l, P:P + B].view(np.uint32), ov[l, P:P + B].view(np.uint32)), f"V layer {l}"
    tok = oracle.argmax(lo)
    for pos in range(P + B, P + B + 2):
        lo = o.forward_x([tok], pos, os_)
        worst = max(worst, assert_logits(g.forward_x([tok], pos, gs), lo, f"decode at {pos}"))
        tok = oracle.argmax(lo)
    print(f"max relative logit difference {worst:.3g}")
