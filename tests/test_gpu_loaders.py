"""safetensors and lm.rs models on the device (TransformerLlamaSt,
transformer_llama_st.rs; TransformerLlamaLmrs, transformer_llama_lmrs.rs):
util::rope in the HF layout, Q8 with f32 group scales of the file's group
size, F16 weights -- prefill and decode logits against the oracle's
restatement of the same loaders, bit for bit, and a chat turn through
infer_ffi."""
from __future__ import annotations

import numpy as np
import pytest

import model_files as MF
from oracle import loaders as L
from oracle import tokenizer as OT
from test_gpu_model import assert_bits

pytestmark = pytest.mark.gpu

MEDIUM = MF.Shape(dim=576, hidden=1536, n_layers=3, n_heads=9, n_kv=3, head_dim=64, ctx=512)

CASES = {
    "st_f16": lambda d: MF.write_safetensors(d, MF.Shape(), seed=1),
    "st_q8_gs64": lambda d: MF.write_safetensors(d, MF.Shape(), q8_gs=64, seed=2),
    "st_q8_gs32_bin": lambda d: MF.write_safetensors(d, MF.Shape(), q8_gs=32, seed=3, tokenizer="bin"),
    "lmrs_gs32": lambda d: MF.write_lmrs(d, MF.Shape(), gs=32, seed=4),
    "lmrs_gs64": lambda d: MF.write_lmrs(d, MF.Shape(), gs=64, seed=5),
    "lmrs_gs192_medium": lambda d: MF.write_lmrs(d, MEDIUM, gs=192, seed=6, n_pad=600),
    "st_q8_medium": lambda d: MF.write_safetensors(d, MEDIUM, q8_gs=64, seed=7),
    "st_f16_medium": lambda d: MF.write_safetensors(d, MEDIUM, seed=8),
    # group size 32 at dim 576: the one-token steps run the 32-block GEMV with
    # 18 blocks per row (a partial last slot) and q/k rows in RoPE pair order
    "lmrs_gs32_medium": lambda d: MF.write_lmrs(d, MEDIUM, gs=32, seed=9, n_pad=600),
    # group size 128: four blocks per group on the GEMV (and the tile kernel
    # for prompts)
    "lmrs_gs128": lambda d: MF.write_lmrs(d, MF.Shape(), gs=128, seed=10),
    "st_q8_gs128_medium": lambda d: MF.write_safetensors(d, MF.Shape(dim=512, hidden=1536, n_layers=2, n_heads=8,
                                                                     n_kv=2, head_dim=64, ctx=512),
                                                         q8_gs=128, seed=11),
}


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    root = tmp_path_factory.mktemp("loaders")
    cache = {}

    def get(name):
        if name not in cache:
            cache[name] = CASES[name](str(root / name))
        return cache[name]
    return get


def _oracle(path, max_ctx_len=0xFFFFFFFF):
    return (L.load_lmrs if path.endswith(".lmrs") else L.load_safetensors)(path, max_ctx_len)


@pytest.mark.parametrize("name,prompt_len,steps", [("st_f16", 20, 8), ("st_f16", 97, 3), ("st_q8_gs64", 20, 8),
                                                    ("st_q8_gs64", 130, 3), ("st_q8_gs32_bin", 33, 5),
                                                    ("lmrs_gs32", 20, 8), ("lmrs_gs32", 64, 4),
                                                    ("lmrs_gs64", 41, 6), ("lmrs_gs192_medium", 70, 4),
                                                    ("st_q8_medium", 50, 4), ("st_f16_medium", 45, 3),
                                                    ("lmrs_gs32_medium", 37, 5), ("lmrs_gs128", 30, 6),
                                                    ("st_q8_gs128_medium", 45, 4)])
def test_model_matches_oracle(gpu, files, name, prompt_len, steps):
    import yallma3_mini_inference_amd as Y
    path = files(name)
    print(f"[loaders] {name} prompt {prompt_len} steps {steps}", flush=True)
    g = Y.load_transformer(path)
    o, _ = _oracle(path)
    assert g.name() == ("TransformerLlamaLmrs" if path.endswith(".lmrs") else "TransformerLlamaSt")
    rng = np.random.default_rng(prompt_len * 3 + len(name))
    prompt = rng.integers(0, o.vocab, prompt_len).astype(np.uint32)
    gs, os_ = g.create_session(), o.create_session()
    assert_bits(g.forward_x(prompt, 0, gs), lo := o.forward_x(prompt, 0, os_), f"{name} prefill")
    tok = int(np.argmax(lo))
    for i in range(steps):
        lo = o.forward_x(np.array([tok], np.uint32), prompt_len + i, os_)
        assert_bits(g.forward_x(np.array([tok], np.uint32), prompt_len + i, gs), lo, f"{name} step {i}")
        tok = int(np.argmax(lo))


@pytest.mark.parametrize("name", ["st_q8_gs64", "lmrs_gs32", "st_f16"])
def test_rerun_without_reset(gpu, files, name):
    """The same prompt twice without a reset: Q8 K/V accumulate (`+=`,
    matmul_q8_slices), F16 K/V are assigned -- as in the oracle."""
    import yallma3_mini_inference_amd as Y
    path = files(name)
    g = Y.load_transformer(path)
    o, _ = _oracle(path)
    prompt = np.arange(3, 40, dtype=np.uint32)
    gs, os_ = g.create_session(), o.create_session()
    for k in range(2):
        assert_bits(g.forward_x(prompt, 0, gs), o.forward_x(prompt, 0, os_), f"{name} run {k}")


def test_capped_context_changes_rope(gpu, files):
    """util::rope scales frequencies by the model's (capped) context length."""
    import yallma3_mini_inference_amd as Y
    path = files("lmrs_gs32")
    g = Y.load_transformer(path, max_ctx_len=64)
    o, _ = _oracle(path, 64)
    assert g.max_ctx_len() == 64
    prompt = np.arange(5, 45, dtype=np.uint32)
    a = g.forward_x(prompt, 0, g.create_session())
    assert_bits(a, o.forward_x(prompt, 0, o.create_session()), "capped")
    full = Y.load_transformer(path)
    assert not np.array_equal(a, full.forward_x(prompt, 0, full.create_session()))


@pytest.mark.parametrize("name", ["lmrs_gs32", "st_q8_gs64"])
def test_infer_ffi_matches_oracle(gpu, files, name):
    import yallma3_mini_inference_amd as Y
    from test_gpu_generate import oracle_conversation
    path = files(name)
    o, otok = _oracle(path)
    prompts = ["Hello world, the quick brown fox", "the lazy dog"]
    assert Y.load_transformer_ffi(path)
    Y.infer_set_max_tokens(10)
    try:
        got = [Y.infer_ffi(p) for p in prompts]
    finally:
        Y.infer_set_max_tokens(0)
        Y.infer_reset()
    want, _ = oracle_conversation(o, otok, prompts, 10)
    assert got == want


def test_load_errors(gpu, tmp_path, files):
    import yallma3_mini_inference_amd as Y
    bad = tmp_path / "bad"
    bad.mkdir()
    p = bad / "model.lmrs"
    MF.llama2c_tokenizer_bin(str(bad / "tokenizer.bin"))
    p.write_bytes(b"nope" + bytes(300))
    with pytest.raises(Y.YlError, match="lm.rs"):
        Y.load_transformer(str(p))
    with pytest.raises(Y.YlError, match="config.json"):
        Y.load_transformer(str(tmp_path / "model.safetensors"))
    with pytest.raises(Y.YlError, match="StSeq"):
        Y.load_transformer(files("st_f16"), sequential=True)
    assert not Y.load_transformer_ffi(str(p))
