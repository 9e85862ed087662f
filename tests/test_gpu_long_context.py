"""Long contexts through the product ABI and the decode graphs.

A GGUF whose llama.context_length is 131072 (every Llama-3.x file's) loads
through load_transformer_ffi (lib.rs:135-152 passes u32::MAX as max_ctx_len,
so the cache is sized to the full context, transformer_llama_gguf.rs:229-233).
Decode steps are captured per context bucket; past 16384 positions the
softmax row streams through LDS in segments.  Prompt batches of 2..63 tokens
whose score row does not fit k_attention's LDS take the tiled path.  The KV
cache below the tested positions is random-filled identically in the device
session and the oracle's (the oracle's cache arrays are writable), so only
the positions under test are computed.  Bar: bit-exact logits, identical
greedy tokens."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def assert_bits(a, b, what=""):
    a = np.ascontiguousarray(a, np.float32).ravel()
    b = np.ascontiguousarray(b, np.float32).ravel()
    bad = np.nonzero(a.view(np.uint32) != b.view(np.uint32))[0]
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first {bad[:4]}: {a[bad[:4]]} vs {b[bad[:4]]}"


def _models(oracle, model_dir, name):
    from yallma3_mini_inference_amd import Transformer, synth
    path = synth.ensure(name, model_dir)
    return Transformer(path), oracle.Model(path), path


def _fill_kv(sessions, oracle_session, P, seed):
    """Same random K/V at positions < P in every device session and the oracle's."""
    m = oracle_session.model
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((m.n_layers, P, m.kv_dim), dtype=np.float32)
    v = rng.standard_normal((m.n_layers, P, m.kv_dim), dtype=np.float32)
    oracle_session.key_cache()[:, :P] = k
    oracle_session.value_cache()[:, :P] = v
    for s in sessions:
        s.upload_kv(k, v)


def test_ffi_loads_long_context_gguf_and_replaces_model(gpu, model_dir):
    import ctypes as C
    from yallma3_mini_inference_amd import synth
    from yallma3_mini_inference_amd._lib import Shape, last_error
    from yallma3_mini_inference_amd.transformer import load_transformer_ffi
    L = gpu.lib()
    long_path, short_path = synth.ensure("tiny_ctx131k", model_dir), synth.ensure("tiny", model_dir)
    assert load_transformer_ffi(long_path) is True, last_error()
    h1 = L.yl_ffi_model()
    assert h1
    sh = Shape()
    gpu.check(L.yl_model_shape(h1, C.byref(sh)))
    assert (sh.ctx_len, sh.dimension, sh.n_heads, sh.n_kv_heads) == (131072, 256, 4, 2)
    # a failed load leaves the current model in place (lib.rs:145-151)
    assert load_transformer_ffi(long_path + ".missing.gguf") is False
    assert L.yl_ffi_model() == h1
    assert load_transformer_ffi(short_path) is True
    h2 = L.yl_ffi_model()
    assert h2 and h2 != h1
    gpu.check(L.yl_model_shape(h2, C.byref(sh)))
    assert (sh.ctx_len, sh.dimension) == (256, 128)


def test_decode_past_16k_positions(gpu, oracle, model_dir):
    """Steps at 16380..16387 cross from the 16384 bucket into the 32768 one
    (segmented softmax); a greedy run over the same positions replays both
    graphs; then a 20-token prompt at 16388 takes the tiled prompt path."""
    g, o, _ = _models(oracle, model_dir, "tiny_ctx131k")
    assert g.max_ctx_len() == 131072
    P = 16380
    gs, gs2, os_ = g.create_session(), g.create_session(), o.create_session()
    _fill_kv((gs, gs2), os_, P, seed=16380)
    tok, ref = 7, []
    for pos in range(P, P + 8):
        lg, lo = g.forward_x([tok], pos, gs), o.forward_x([tok], pos, os_)
        assert_bits(lg, lo, f"decode at {pos}")
        tok = oracle.argmax(lo)
        ref.append(tok)
    toks = g.generate_greedy(gs2, 7, P, 8)
    assert list(toks) == ref
    rng = np.random.default_rng(20)
    prompt = rng.integers(0, o.vocab, 20).astype(np.uint32)
    assert_bits(g.forward_x(prompt, P + 8, gs), o.forward_x(prompt, P + 8, os_), "20-token prompt at 16388")
    n = P + 28
    assert_bits(gs.key_cache()[:, P:n], os_.key_cache()[:, P:n], "K cache")
    assert_bits(gs.value_cache()[:, P:n], os_.value_cache()[:, P:n], "V cache")


def test_decode_bound_of_head_size_32(gpu, oracle, model_dir):
    """Head size 32 keeps the scores row in LDS: decode reaches 16384
    positions and reports YL_ERR_RANGE past them; prompts go further."""
    from yallma3_mini_inference_amd import YlError
    g, o, _ = _models(oracle, model_dir, "tiny_hd32_long")
    gs, os_ = g.create_session(), o.create_session()
    P = 16383
    _fill_kv((gs,), os_, P, seed=32)
    assert_bits(g.forward_x([3], P, gs), o.forward_x([3], P, os_), "decode at 16383")
    with pytest.raises(YlError) as ei:
        g.forward_x([3], P + 1, gs)
    assert ei.value.status == -8
    with pytest.raises(YlError):
        g.generate_greedy(gs, 3, P, 2)
    prompt = np.array([5, 9, 11, 2], np.uint32)
    assert_bits(g.forward_x(prompt, P + 1, gs), o.forward_x(prompt, P + 1, os_), "prompt at 16384")


def test_split_decode_attention_in_graph(gpu, oracle, model_dir):
    """ctx 8448 (bucket 8448): decode at 5000+ runs k_attn_scores, softmax,
    P.V by lane and the output kernel inside the decode graph with seq well
    below the bucket's size; earlier positions use the 4096 bucket."""
    g, o, _ = _models(oracle, model_dir, "tiny_8k")
    gs, gs2, os_ = g.create_session(), g.create_session(), o.create_session()
    P = 5000
    _fill_kv((gs, gs2), os_, P, seed=5000)
    tok, ref = 11, []
    for pos in range(P, P + 4):
        lo = o.forward_x([tok], pos, os_)
        assert_bits(g.forward_x([tok], pos, gs), lo, f"decode at {pos}")
        tok = oracle.argmax(lo)
        ref.append(tok)
    for i in range(6):
        tok = oracle.argmax(o.forward_x([tok], P + 4 + i, os_))
        ref.append(tok)
    assert list(g.generate_greedy(gs2, 11, P, 10)) == ref
    # a short context on the same model: the 4096 bucket's single kernel
    gs3, os3 = g.create_session(), o.create_session()
    prompt = np.array([1, 2, 3, 4, 5, 6, 7, 8, 9], np.uint32)
    assert_bits(g.forward_x(prompt, 0, gs3), lo := o.forward_x(prompt, 0, os3), "prompt")
    tok = oracle.argmax(lo)
    for pos in range(9, 13):
        lo = o.forward_x([tok], pos, os3)
        assert_bits(g.forward_x([tok], pos, gs3), lo, f"short decode at {pos}")
        tok = oracle.argmax(lo)
