"""Pins the oracle's tokenizer and sampler restatement (oracle/tokenizer.py)
with checks that do not reuse its formulas: hand-worked pieces and merges,
the Hugging Face `tokenizers` BPE model on a trained vocabulary, the Unicode
standard's replacement examples, a second xorshift64* implementation in
numpy, and sampler outcomes worked out by hand (tokenizer.rs, sampler.rs)."""
from __future__ import annotations

import numpy as np
import pytest

import bpe_vocab
from oracle import tokenizer as OT


@pytest.mark.parametrize("text,pieces", [
    ("Hello world's  test", ["Hello", " world", "'s", "  ", "test"]),
    ("I'm'S", ["I", "'m", "'", "S"]),
    ("we'll they've you're", ["we", "'ll", " they", "'ve", " you", "'re"]),
    ("abc123def", ["abc", "123", "def"]),
    (" \n x", [" \n ", "x"]),                       # no (?!\S): the run takes the last space too
    ("x y", ["x", " ", "y"]),             # NO-BREAK SPACE is White_Space
    ("!\x1c", ["!\x1c"]),                           # U+001C is not White_Space (it is for str.isspace)
    ("٣٤ Ⅻ ½", ["٣٤", " Ⅻ", " ½"]),   # Nd, Nl, No
    ("日本語テキスト", ["日本語テキスト"]),
    ("\U0001F600\U0001F600 ok", ["\U0001F600\U0001F600", " ok"]),
    ("a  ,b", ["a", "  ", ",", "b"]),
])
def test_split_hand_cases(text, pieces):
    assert OT.gpt2_split(text) == pieces


def _tok(vocab, merges, **kw):
    return OT.OracleTokenizer(vocab, merges, 0, 1, **kw)


def test_bpe_hand_cases():
    vocab = ["a", "b", "c", "d", "ab", "bc", "abc", "cd", "x", "dx"]
    t = _tok(vocab, ["a b", "b c", "ab c", "c d"])
    ids = lambda s: [vocab[i] for i in t.encode(s)]
    assert ids("abc") == ["abc"]            # ab (rank 0) first, then ab+c
    assert ids("bcd") == ["bc", "d"]        # bc outranks cd; "bcd" is no token
    assert ids("abab") == ["ab", "ab"]      # equal scores: the first pair merges first
    assert ids("dx") == ["dx"]              # a token from no merge has score 0 and still merges
    # the merged text's score decides, whichever pair forms it: with "b c" ranked
    # first, a + bc -> "abc" (a rank-ordered BPE would stop at [a, bc])
    t2 = _tok(vocab, ["b c", "a b", "ab c"])
    assert [vocab[i] for i in t2.encode("abc")] == ["abc"]


def test_bpe_matches_hf_on_trained_vocabulary():
    tokens, merges, hf = bpe_vocab.train()
    t = OT.OracleTokenizer(tokens, merges, 0, 1, pre="gpt2")
    table = OT.gpt2_byte_table()
    n = 0
    for text in bpe_vocab.CORPUS[:12] + ["unseen words: zebra xylophone quizzical", "über-naïve café 2025"]:
        for seg in OT.gpt2_split(text):
            mine = t.bpe_merge([t.byte_to_token[b] for b in seg.encode()])
            ref = bpe_vocab.hf_bpe_segment(hf, "".join(table[b] for b in seg.encode()))
            if mine != ref:
                # the only allowed difference: HF stopped where a neighbouring
                # pair's concatenation is still a vocabulary text
                assert any(tokens[ref[k]] + tokens[ref[k + 1]] in t.index for k in range(len(ref) - 1)), seg
            n += 1
    assert n > 200


@pytest.mark.parametrize("raw,text", [
    (b"\xe2\x82A", "�A"),                      # truncated sequence: one U+FFFD
    (b"\xf0\x80\x80", "���"),        # F0 80: invalid second byte
    (b"\xed\xa0\x80", "���"),        # a surrogate
    (b"\xc0\xaf", "��"),                  # overlong
    (b"\xf4\x90\x80\x80", "�" * 4),            # beyond U+10FFFF
    (b"ok\xe2\x82", "ok�"),                    # incomplete at the end
    (b"\xe2\x82\xac", "€"),
])
def test_decode_lossy_unicode_examples(raw, text):
    table = OT.gpt2_byte_table()
    vocab = [table[b] for b in range(256)]
    t = _tok(vocab, [])
    assert t.decode(list(raw)) == text


def test_decode_special_token_text():
    table = OT.gpt2_byte_table()
    vocab = [table[b] for b in range(256)] + ["<|eot_id|>", "␀x"]
    t = _tok(vocab, [])
    assert t.decode([256]) == "<|eot_id|>"          # every character maps back through the byte table
    assert t.decode([257]) == "␀x"            # characters outside the table keep their UTF-8
    assert t.decode([9999]) == ""                   # out-of-range ids are skipped


def test_chatml_template_text():
    tmpl = ("{% for message in messages %}{% if loop.first and messages[0]['role'] != 'system' %}"
            "{{ '<|im_start|>system\\nBe brief.<|im_end|>\\n' }}{% endif %}"
            "{{'<|im_start|>' + message['role'] + '\\n' + message['content'] + '<|im_end|>' + '\\n'}}{% endfor %}"
            "{% if add_generation_prompt %}{{ '<|im_start|>assistant\\n' }}{% endif %}")
    tokens, merges, _ = bpe_vocab.train()
    t = OT.OracleTokenizer(tokens, merges, 0, 1, pre="gpt2", chat_template=tmpl)
    got = t.decode(t.apply_turn_template("hi", True))
    assert got == ("<|im_start|>system\nBe brief.<|im_end|>\n<|im_start|>user\nhi<|im_end|>\n"
                   "<|im_start|>assistant\n<|im_end|>\n<|im_start|>assistant\n")


def test_random_f32_second_implementation():
    for seed in (0, 1, 42, 12345, 2 ** 63 + 11):
        s = np.array([seed], np.uint64)
        with np.errstate(over="ignore"):
            s ^= s >> np.uint64(12)
            s ^= s << np.uint64(25)
            s ^= s >> np.uint64(27)
            r = (s * np.uint64(0x2545F4914F6CDD1D)) >> np.uint64(32)
        want = np.float32(int(r[0]) >> 8) / np.float32(2 ** 24)
        assert OT.random_f32(seed) == want


def _logits(p):
    return np.log(np.maximum(np.asarray(p, np.float64), 1e-13)).astype(np.float32)


def test_sampler_hand_cases():
    assert OT._argmax_first(np.array([1, 3, 3, 2], np.float32)) == 1
    assert OT.OracleSampler(4, 0.0, 0.9, 42).sample(np.array([1, 3, 3, 2], np.float32)) == 1
    # top-p 0.7 over [0.2, 0.5, 0.3]: sorted 0.5, 0.3 (cum 0.8 > 0.7 stops), r = rand * 0.8
    assert 0.33 < OT.random_f32(42) < 0.34          # r = 0.27 < 0.5 -> the 0.5 entry
    assert OT.OracleSampler(3, 1.0, 0.7, 42).sample(_logits([0.2, 0.5, 0.3])) == 1
    assert 0.91 < OT.random_f32(19) < 0.92          # r = 0.73 in (0.5, 0.8] -> the 0.3 entry
    assert OT.OracleSampler(3, 1.0, 0.7, 19).sample(_logits([0.2, 0.5, 0.3])) == 2
    # multinomial (top_p >= 1): first cdf above rand; rand(42) = 0.339 -> cdf 0.2, 0.7
    assert OT.OracleSampler(3, 1.0, 1.0, 42).sample(_logits([0.2, 0.5, 0.3])) == 1


def test_sampler_stale_entries():
    """sample_topp sorts the whole persistent array (sampler.rs:122): entries
    left from an earlier call can outrank this call's candidates."""
    s = OT.OracleSampler(4, 1.0, 0.95, 19)          # rand 0.918
    s.sample(_logits([0.25, 0.25, 0.25, 0.25]))
    # candidates 0.9, 0.05, 0.05 fill positions 0-2; position 3 keeps (0.25, id 3):
    # sorted 0.9, 0.25(stale) -> cum 1.15, r = 0.918 * 1.15 = 1.06 > 0.9 -> id 3
    assert s.sample(_logits([0.9, 0.05, 0.05, 0.0])) == 3
