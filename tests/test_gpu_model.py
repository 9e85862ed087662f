"""End-to-end parity of the HIP forward path against the oracle on seeded
synthetic GGUF models: prefill logits, every greedy step's logits (bit-exact)
and the greedy token sequence (identical), plus the reference's session
semantics (K/V `+=` on re-runs, reset, out-of-range ids, ctx bound)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def assert_bits(a, b, what=""):
    a = np.ascontiguousarray(a, np.float32).ravel()
    b = np.ascontiguousarray(b, np.float32).ravel()
    bad = np.nonzero(a.view(np.uint32) != b.view(np.uint32))[0]
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first {bad[:4]}: {a[bad[:4]]} vs {b[bad[:4]]}"


def _models(gpu, oracle, model_dir, name):
    from yallma3_mini_inference_amd import Transformer, synth
    path = synth.ensure(name, model_dir)
    return Transformer(path), oracle.Model(path), path


@pytest.mark.parametrize("name,prompt_len,steps", [("tiny", 20, 24), ("tiny_q4", 17, 16), ("tiny_mixed", 33, 20),
                                                    ("tiny_pad", 9, 12), ("tiny", 100, 6), ("tiny_q4", 130, 4),
                                                    ("tiny_mixed", 200, 4), ("tiny_yarn", 40, 12),
                                                    ("tiny_yarn", 100, 6), ("tiny_yarn_q4", 70, 8),
                                                    ("tiny_yarn_q4", 23, 10)])
def test_prefill_then_greedy_decode(gpu, oracle, model_dir, name, prompt_len, steps):
    g, o, _ = _models(gpu, oracle, model_dir, name)
    rng = np.random.default_rng(prompt_len)
    prompt = rng.integers(0, o.vocab, prompt_len).astype(np.uint32)
    gs, os_ = g.create_session(), o.create_session()
    lg, lo = g.forward_x(prompt, 0, gs), o.forward_x(prompt, 0, os_)
    assert_bits(lg, lo, "prefill logits")
    tok = oracle.argmax(lo)
    pos = prompt_len
    for step in range(steps):
        lg, lo = g.forward_x([tok], pos, gs), o.forward_x([tok], pos, os_)
        assert_bits(lg, lo, f"step {step} logits")
        tok = oracle.argmax(lo)
        assert int(np.argmax(lg)) == tok or lg[tok] == lg.max()
        pos += 1
    # device-resident cache equals the oracle's
    assert_bits(gs.key_cache()[:, :pos], os_.key_cache()[:, :pos], "K cache")
    assert_bits(gs.value_cache()[:, :pos], os_.value_cache()[:, :pos], "V cache")


@pytest.mark.parametrize("name", ["tiny", "tiny_mixed", "tiny_yarn"])
def test_generate_greedy_matches_oracle_tokens(gpu, oracle, model_dir, name):
    g, o, _ = _models(gpu, oracle, model_dir, name)
    prompt = (np.arange(12, dtype=np.uint32) * 37) % o.vocab
    os_ = o.create_session()
    lo = o.forward_x(prompt, 0, os_)
    ref = [oracle.argmax(lo)]
    for i in range(30):
        ref.append(oracle.argmax(o.forward_x([ref[-1]], len(prompt) + i, os_)))
    gs = g.create_session()
    first = g.forward_argmax(prompt, 0, gs)
    assert first == ref[0]
    toks = g.generate_greedy(gs, first, len(prompt), 30)
    assert list(toks) == ref[1:]


def test_kv_accumulates_on_rerun_and_reset(gpu, oracle, model_dir):
    # forward.rs:166-169 writes K/V with `+=`; re-running a position changes
    # its logits, exactly as the reference does (simd_tests.rs:474-506).
    g, o, _ = _models(gpu, oracle, model_dir, "tiny")
    gs, os_ = g.create_session(), o.create_session()
    a1, b1 = g.forward_x([5], 0, gs), o.forward_x([5], 0, os_)
    a2, b2 = g.forward_x([5], 0, gs), o.forward_x([5], 0, os_)
    assert_bits(a1, b1, "first run")
    assert_bits(a2, b2, "second run")
    assert not np.array_equal(a1, a2)
    gs.reset()
    assert_bits(g.forward_x([5], 0, gs), b1, "after reset")


def test_out_of_range_token_and_bounds(gpu, oracle, model_dir):
    from yallma3_mini_inference_amd import YlError
    g, o, _ = _models(gpu, oracle, model_dir, "tiny")
    emb = g.get_embeddings_batch([3, o.vocab + 5])
    assert_bits(emb[0], o.embedding().reshape(o.vocab, o.dim)[3], "embedding row")
    assert (emb[1] == 0).all()
    gs, os_ = g.create_session(), o.create_session()
    assert_bits(g.forward_x([1, o.vocab + 9, 2], 0, gs), o.forward_x([1, o.vocab + 9, 2], 0, os_), "oob id")
    with pytest.raises(YlError):
        g.forward_x([1, 2], o.ctx_len - 1, gs)
    with pytest.raises(YlError):
        g.forward_x([], 0, gs)


def test_chunked_prefill_matches_oracle(gpu, oracle, model_dir):
    # a prompt fed in chunks (start_pos > 0, batch > 1) uses the same
    # seq_len-dependent P.V grouping as the reference
    g, o, _ = _models(gpu, oracle, model_dir, "tiny_mixed")
    rng = np.random.default_rng(3)
    toks = rng.integers(0, o.vocab, 50).astype(np.uint32)
    gs, os_ = g.create_session(), o.create_session()
    for a, b in ((0, 11), (11, 30), (30, 31), (31, 50)):
        assert_bits(g.forward_x(toks[a:b], a, gs), o.forward_x(toks[a:b], a, os_), f"chunk {a}:{b}")


def test_smollm2_shape_short(gpu, oracle, model_dir):
    g, o, _ = _models(gpu, oracle, model_dir, "smollm2_135m")
    rng = np.random.default_rng(135)
    prompt = rng.integers(0, o.vocab, 24).astype(np.uint32)
    gs, os_ = g.create_session(), o.create_session()
    assert_bits(g.forward_x(prompt, 0, gs), lo := o.forward_x(prompt, 0, os_), "prefill")
    tok = oracle.argmax(lo)
    toks = g.generate_greedy(gs, tok, 24, 6)
    ref = []
    for i in range(6):
        tok = oracle.argmax(o.forward_x([tok], 24 + i, os_))
        ref.append(tok)
    assert list(toks) == ref


def test_long_context_decode(gpu, oracle, model_dir):
    """ctx 4096: decode steps take the single decode attention kernel, whose
    softmax sum runs on one lane up to 2560 positions and on one wavefront
    (super-rows of 512) beyond; the greedy graph replays the same kernel."""
    g, o, _ = _models(gpu, oracle, model_dir, "tiny_long")
    rng = np.random.default_rng(4096)
    toks = rng.integers(0, o.vocab, 2100).astype(np.uint32)
    gs, os_ = g.create_session(), o.create_session()
    assert_bits(g.forward_x(toks[:30], 0, gs), o.forward_x(toks[:30], 0, os_), "prefill 30")
    for i in range(30, 34):
        assert_bits(g.forward_x(toks[i:i + 1], i, gs), o.forward_x(toks[i:i + 1], i, os_), f"decode at {i}")
    assert_bits(g.forward_x(toks[34:2093], 34, gs), o.forward_x(toks[34:2093], 34, os_), "prefill to 2093")
    for i in range(2093, 2100):
        lo = o.forward_x(toks[i:i + 1], i, os_)
        assert_bits(g.forward_x(toks[i:i + 1], i, gs), lo, f"decode at {i}")
    tok = oracle.argmax(lo)
    toks_g = g.generate_greedy(gs, tok, 2100, 4)
    ref = []
    for i in range(4):
        tok = oracle.argmax(o.forward_x([tok], 2100 + i, os_))
        ref.append(tok)
    assert list(toks_g) == ref


@pytest.mark.parametrize("name,start", [("tiny_yarn", 3000), ("tiny_yarn_q4", 4000)])
def test_yarn_decode_at_high_positions(gpu, oracle, model_dir, name, start):
    # YaRN RoPE scaling and llama.attention.scale (util.rs:653-724,
    # forward.rs:142-146) where the angles are large: a random KV cache below
    # `start` shared by both sides, then single-token steps and a greedy run
    g, o, _ = _models(gpu, oracle, model_dir, name)
    rng = np.random.default_rng(start)
    L, kvd = o.n_layers, o.n_kv_heads * o.head_size
    kc = rng.standard_normal((L, start, kvd), dtype=np.float32)
    vc = rng.standard_normal((L, start, kvd), dtype=np.float32)
    gs, os_ = g.create_session(), o.create_session()
    gs.upload_kv(kc, vc)
    os_.key_cache()[:, :start] = kc
    os_.value_cache()[:, :start] = vc
    tok, pos = 7, start
    for step in range(4):
        lg, lo = g.forward_x([tok], pos, gs), o.forward_x([tok], pos, os_)
        assert_bits(lg, lo, f"step {step} logits")
        tok = oracle.argmax(lo)
        pos += 1
    ref = []
    for i in range(8):
        ref.append(oracle.argmax(o.forward_x([tok if not ref else ref[-1]], pos + i, os_)))
    toks = g.generate_greedy(gs, tok, pos, 8)
    assert list(toks) == ref
    assert_bits(gs.key_cache()[:, :pos + 8], os_.key_cache()[:, :pos + 8], "K cache")
