"""The library's tokenizer, chat templates and sampler (host C++, no GPU)
against the oracle restatement of tokenizer.rs / sampler.rs, on GGUF files
carrying trained byte-level BPE vocabularies."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import pytest

import bpe_vocab
import yallma3_mini_inference_amd as Y
from oracle import tokenizer as OT
from yallma3_mini_inference_amd import synth

CHATML = ("{% for message in messages %}{% if loop.first and messages[0]['role'] != 'system' %}"
          "{{ '<|im_start|>system\\nYou are a helpful AI assistant named SmolLM, trained by Hugging Face<|im_end|>\\n' }}"
          "{% endif %}{{'<|im_start|>' + message['role'] + '\\n' + message['content'] + '<|im_end|>' + '\\n'}}"
          "{% endfor %}{% if add_generation_prompt %}{{ '<|im_start|>assistant\\n' }}{% endif %}")

# the structure of Llama 3.2's template (tool branches left out)
LLAMA32 = """{{- bos_token }}
{%- if custom_tools is defined %}
    {%- set tools = custom_tools %}
{%- endif %}
{%- if not tools_in_user_message is defined %}
    {%- set tools_in_user_message = true %}
{%- endif %}
{%- if not date_string is defined %}
    {%- if strftime_now is defined %}
        {%- set date_string = strftime_now("%d %b %Y") %}
    {%- else %}
        {%- set date_string = "26 Jul 2024" %}
    {%- endif %}
{%- endif %}
{%- if not tools is defined %}
    {%- set tools = none %}
{%- endif %}

{#- This block extracts the system message, so we can slot it into the right place. #}
{%- if messages[0]['role'] == 'system' %}
    {%- set system_message = messages[0]['content']|trim %}
    {%- set messages = messages[1:] %}
{%- else %}
    {%- set system_message = "" %}
{%- endif %}

{#- System message #}
{{- "<|start_header_id|>system<|end_header_id|>\\n\\n" }}
{%- if tools is not none %}
    {{- "Environment: ipython\\n" }}
{%- endif %}
{{- "Cutting Knowledge Date: December 2023\\n" }}
{{- "Today Date: " + date_string + "\\n\\n" }}
{{- system_message }}
{{- "<|eot_id|>" }}

{%- for message in messages %}
    {%- if not (message.role == 'ipython' or message.role == 'tool' or 'tool_calls' in message) %}
        {{- '<|start_header_id|>' + message['role'] + '<|end_header_id|>\\n\\n'+ message['content'] | trim + '<|eot_id|>' }}
    {%- endif %}
{%- endfor %}
{%- if add_generation_prompt %}
    {{- '<|start_header_id|>assistant<|end_header_id|>\\n\\n' }}
{%- endif %}
"""

TEXTS = [
    "Hello, world! It's a small world, isn't it?",
    "The quick brown fox jumps over the lazy dog.",
    "  leading and trailing spaces  ",
    "Numbers 3.14159 and 2024, 100% sure",
    "über café naïve — “quotes” © 2025",
    "中文 文本 日本語 テキスト 한국어",
    "emoji 😀 🚀 and ★ → ✓",
    "tabs\tand\nnew\n\nlines",
    "<|im_start|> a special-looking text <|im_end|>",
    "x",
    "unseen: zebra xylophone quizzical",
]


def llama_vocab(tokens):
    """A 128256-entry vocabulary: the trained tokens, fillers no merge can
    form (their first character is outside the byte table), then the
    Llama-3 special tokens at 128000..128255."""
    v = list(tokens) + [f"␀{i}" for i in range(128000 - len(tokens))]
    names = {0: "<|begin_of_text|>", 1: "<|end_of_text|>", 6: "<|start_header_id|>", 7: "<|end_header_id|>",
             8: "<|eom_id|>", 9: "<|eot_id|>"}
    v += [names.get(k, f"<|reserved_special_token_{k}|>") for k in range(256)]
    return v


VARIANTS = {
    "gpt2": dict(pre="gpt2"),
    "smollm_space": dict(pre="smollm", add_space_prefix=True),
    "default": dict(pre=None),
    "gpt2_chatml": dict(pre="gpt2", chat_template=CHATML),
    "gpt2_no_bos": dict(pre="gpt2", add_bos_token=False),
    "llama_plain": dict(pre="gpt2", llama=True),
    "llama32_template": dict(pre="gpt2", llama=True, chat_template=LLAMA32),
}


@pytest.fixture(scope="module")
def trained():
    return bpe_vocab.train()


@pytest.fixture(scope="module")
def ggufs(tmp_path_factory, trained):
    tokens, merges, _ = trained
    d = tmp_path_factory.mktemp("tok")
    out = {}
    for name, kw in VARIANTS.items():
        kw = dict(kw)
        llama = kw.pop("llama", False)
        vocab = llama_vocab(tokens) if llama else tokens
        bos, eos = (128000, 128009) if llama else (0, 1)
        spec = synth.TokenizerSpec(tuple(vocab), tuple(merges), bos, eos, **kw)
        cfg = synth.ModelConfig(64, 128, 1, 2, 1, len(vocab), 256)
        path = synth.write(str(d / f"{name}.gguf"), cfg, spec)
        oracle = OT.OracleTokenizer(vocab, merges, bos, eos, pre=kw.get("pre") or "default",
                                    add_bos_token=kw.get("add_bos_token", True) is not False,
                                    add_space_prefix=bool(kw.get("add_space_prefix")),
                                    chat_template=kw.get("chat_template"))
        out[name] = (path, oracle)
    return out


def test_pretokenize_matches_oracle():
    rng = np.random.default_rng(0)
    pool = list("ab xyz'stlvrmdAB  \t\n0123456789.,!?-_()") + ["é", "ü", " ", "—", "中", "😀", "٣", "Ⅻ", "½",
                                                                "\x1c", " ", "’", "ʼ"]
    texts = list(TEXTS) + ["".join(rng.choice(pool, size=int(rng.integers(1, 40)))) for _ in range(300)]
    for t in texts:
        assert Y.pretokenize(t) == OT.gpt2_split(t), repr(t)


@pytest.mark.parametrize("variant", list(VARIANTS))
def test_encode_decode_match_oracle(ggufs, variant):
    path, o = ggufs[variant]
    t = Y.Tokenizer.from_gguf(path)
    assert t.vocab_size == len(o.vocab)
    for text in TEXTS:
        for bos, eos in ((False, False), (True, False), (True, True)):
            ids = t.encode(text, bos, eos)
            assert ids == o.encode(text, bos, eos), (text, bos, eos)
        ids = t.encode(text)
        assert t.decode(ids) == o.decode(ids) == (" " + text if o.add_space_prefix and not text.startswith(" ")
                                                   else text)
    rng = np.random.default_rng(1)
    for _ in range(50):   # arbitrary id strings, including invalid UTF-8 byte sequences
        ids = rng.integers(0, min(len(o.vocab), 800), size=int(rng.integers(1, 12))).tolist()
        assert t.decode(ids) == o.decode(ids)


@pytest.mark.parametrize("variant", list(VARIANTS))
def test_templates_match_oracle(ggufs, variant):
    path, o = ggufs[variant]
    t = Y.Tokenizer.from_gguf(path)
    for text in ("", "You are terse.", "  padded system  "):
        assert t.apply_system_template(text) == o.apply_system_template(text), text
    for text in ("hi", "What is 2+2?", " spaced \n"):
        for flag in (True, False):
            assert t.apply_turn_template(text, flag) == o.apply_turn_template(text, flag), (text, flag)
        assert t.chat_prompt(text) == o.chat_prompt(text), text
        assert t.encode_wrap_n_header(text, True) == o.encode_wrap_n_header(text, "", True)


def test_llama_turn_layout(ggufs):
    """Without a chat template, a Llama-3 vocabulary gets the header-id turn
    layout (tokenizer.rs:526-540)."""
    path, o = ggufs["llama_plain"]
    t = Y.Tokenizer.from_gguf(path)
    turn = t.apply_turn_template("hi", True)
    u, a = o.encode("user"), o.encode("assistant")
    assert turn == [128006, u[0], 128007, 271] + o.encode("hi") + [128009, 128006, a[0], 128007, 271]
    assert t.apply_system_template("") == [128000, 128006] + o.encode("system") + [128007, 271, 271, 128009]


def test_tokenizer_errors(ggufs):
    path, _ = ggufs["gpt2"]
    t = Y.Tokenizer.from_gguf(path)
    with pytest.raises(Y.YlError):
        t.encode("")                       # tokenizer.rs:326 asserts non-empty text
    n = C.c_size_t()
    buf = np.zeros(8, np.uint32)
    assert Y.lib().yl_tokenize(t._h, b"\xff\xfe", 0, 0, buf.ctypes.data, 8, C.byref(n)) == -1
    with pytest.raises(Y.YlError):
        Y.Tokenizer.from_gguf(os.path.join(os.path.dirname(path), "missing.gguf"))


def test_template_errors_are_reported(tmp_path, trained):
    tokens, merges, _ = trained
    cfg = synth.ModelConfig(64, 128, 1, 2, 1, len(tokens), 256)
    for tmpl in ("{{ messages[0]['content'].strip() }}",      # no Python methods without pycompat
                 "{{ undefined_value.attr }}",                 # attribute of an undefined value
                 "{% for m in messages %}"):                   # syntax error
        p = synth.write(str(tmp_path / "bad.gguf"), cfg, synth.TokenizerSpec(tuple(tokens), tuple(merges), 0, 1,
                                                                            pre="gpt2", chat_template=tmpl))
        t = Y.Tokenizer.from_gguf(p)
        with pytest.raises(Y.YlError, match="chat template"):
            t.apply_turn_template("hi", True)


@pytest.mark.parametrize("temperature,top_p", [(0.0, 0.9), (0.7, 0.9), (1.0, 1.0), (0.5, 0.5), (1.3, 0.0),
                                               (0.7, 0.2)])
def test_sampler_matches_oracle(temperature, top_p):
    rng = np.random.default_rng(int(temperature * 10 + top_p * 100))
    V = 1000
    s = Y.Sampler(V, temperature, top_p, 42)
    o = OT.OracleSampler(V, temperature, top_p, 42)
    for step in range(6):
        logits = (rng.standard_normal(V) * (1 + step)).astype(np.float32)
        a = logits.copy()
        got = s.sample(a)
        assert got == o.sample(logits), step
    # seeds whose draw lands elsewhere in the distribution
    for seed in (3, 19, 35):
        logits = rng.standard_normal(V).astype(np.float32)
        assert Y.Sampler(V, temperature, top_p, seed).sample(logits.copy()) == \
            OT.OracleSampler(V, temperature, top_p, seed).sample(logits)


def test_sampler_keeps_stale_entries():
    """The reference's persistent candidate array (sampler.rs:122)."""
    s = Y.Sampler(4, 1.0, 0.95, 19)
    s.sample(np.log(np.full(4, 0.25, np.float32)))
    assert s.sample(np.log(np.array([0.9, 0.05, 0.05, 1e-13], np.float32))) == 3


def test_sampler_rewrites_logits_in_place():
    logits = np.array([1.0, 2.0, 3.0], np.float32)
    Y.Sampler(3, 0.5, 1.0, 42).sample(logits)
    e = np.exp(np.float64([2.0, 4.0, 6.0]) - 6.0)
    np.testing.assert_allclose(logits, e / e.sum(), rtol=1e-6)
