"""Text generation through the product ABI: infer_ffi over a conversation
(main.rs:161-219 semantics, README.md:81-92) and Transformer.generate_text,
against the oracle's forward pass + the oracle tokenizer and sampler."""
from __future__ import annotations

import numpy as np
import pytest

import bpe_vocab
import yallma3_mini_inference_amd as Y
from oracle import oracle as O
from oracle import tokenizer as OT
from test_tokenizer import CHATML
from yallma3_mini_inference_amd import synth

pytestmark = pytest.mark.gpu

MAX_TOKENS = 12


@pytest.fixture(scope="module")
def chat_model(tmp_path_factory):
    tokens, merges, _ = bpe_vocab.train()
    spec = synth.TokenizerSpec(tuple(tokens), tuple(merges), 0, 1, pre="gpt2", chat_template=CHATML)
    cfg = synth.ModelConfig(128, 256, 2, 4, 2, len(tokens), 256, seed=5)
    path = synth.write(str(tmp_path_factory.mktemp("chat") / "chat.gguf"), cfg, spec)
    otok = OT.OracleTokenizer(tokens, merges, 0, 1, pre="gpt2", chat_template=CHATML)
    return path, otok


def oracle_conversation(model, otok, prompts, max_tokens, temperature=0.7, top_p=0.9, seed=42):
    """The CLI loop (main.rs:148-216) on the oracle: one session and sampler.
    `model` is a GGUF path or an oracle Model."""
    m = O.Model(model) if isinstance(model, str) else model
    s = m.create_session()
    smp = OT.OracleSampler(len(otok.vocab), temperature, top_p, seed)
    pos, texts, ids_all = 0, [], []
    for k, p in enumerate(prompts):
        prompt = (otok.chat_prompt(p) if k == 0 else
                  otok.apply_turn_template(p.strip(OT.RUST_WHITE_SPACE), True))
        logits = m.forward_x(np.array(prompt, np.uint32), pos, s)
        pos += len(prompt)
        nxt = smp.sample(logits)
        out, ids, gen = "", [], 0
        while nxt != otok.eos and pos < m.ctx_len and gen < max_tokens:
            out += otok.decode([nxt])
            ids.append(nxt)
            logits = m.forward_x(np.array([nxt], np.uint32), pos, s)
            pos += 1
            gen += 1
            nxt = smp.sample(logits)
        texts.append(out)
        ids_all.append(ids)
    return texts, ids_all


def test_infer_ffi_conversation_matches_oracle(chat_model):
    path, otok = chat_model
    prompts = ["Hello there, who are you?", "  And what about the fox?  "]
    assert Y.load_transformer_ffi(path)
    Y.infer_set_max_tokens(MAX_TOKENS)
    try:
        got = [Y.infer_ffi(p) for p in prompts]
    finally:
        Y.infer_set_max_tokens(0)
        Y.infer_reset()
    want, _ = oracle_conversation(path, otok, prompts, MAX_TOKENS)
    assert got == want


def test_infer_ffi_errors(chat_model):
    path, _ = chat_model
    assert Y.load_transformer_ffi(path)
    assert Y.infer_ffi("   ") is None            # the CLI skips empty input
    assert "empty" in Y._lib.last_error()


def test_generate_text_matches_oracle_and_greedy(chat_model):
    path, otok = chat_model
    g = Y.Transformer(path)
    tok = g.tokenizer()
    prompt = tok.chat_prompt("Tell me about the quick brown fox.")
    assert prompt == otok.chat_prompt("Tell me about the quick brown fox.")
    # sampled (temperature 0.7, top-p 0.9)
    s = g.create_session()
    text, ids = g.generate_text(s, Y.Sampler(g.vocab_size(), 0.7, 0.9, 42), prompt, max_tokens=16)
    want_text, want_ids = oracle_conversation(path, otok, ["Tell me about the quick brown fox."], 16)
    assert (text, ids) == (want_text[0], want_ids[0])
    assert s.pos == len(prompt) + len(ids)
    # greedy: the same tokens as the device argmax chain
    s2 = g.create_session()
    text0, ids0 = g.generate_text(s2, Y.Sampler(g.vocab_size(), 0.0, 0.9, 42), prompt, max_tokens=10)
    s3 = g.create_session()
    first = g.forward_argmax(np.array(prompt, np.uint32), 0, s3)
    chain = [first] + list(g.generate_greedy(s3, first, len(prompt), 9))
    n = len(ids0)
    assert ids0 == chain[:n]
    assert n == 10 or chain[n] == g.eos_token()
    assert text0 == tok.decode(ids0)
