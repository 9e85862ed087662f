"""CPU restatement of the reference's tokenizer and sampler.

TEST INFRASTRUCTURE ONLY (imported by tests/, never by the product package).
Each function names the reference code it restates (paths relative to the
reference repository).  It shares no code with the library's C++ tokenizer:
the GPT-2 split is the `regex` module running the reference's pattern (with
\\s spelled \\p{White_Space}, which is what the Rust regex crate's Unicode \\s
means), chat templates render with jinja2, and the softmax uses the C
library's expf as Rust's f32::exp does.

Pinned by tests/test_tokenizer_oracle.py: the split against hand-listed
pieces, BPE against the Hugging Face `tokenizers` byte-level BPE on a trained
vocabulary and against hand-worked merge cases, decode against Python's UTF-8
decoder (errors="replace"), templates against hand-written expected text, and
the sampler against closed forms (argmax, a known xorshift64* value, cdf
crossings worked by hand, the stale-entry quirk).
"""
from __future__ import annotations

import ctypes
import json
import struct

import jinja2
import numpy as np
import regex

# tokenizer.rs:29-31, with \s as the Unicode White_Space property
GPT2_PATTERN = regex.compile(
    r"'(?:[sdmt]|ll|ve|re)| ?\p{L}+| ?\p{N}+| ?[^\p{White_Space}\p{L}\p{N}]+|\p{White_Space}+")

BEGIN_OF_TEXT, START_HEADER, END_HEADER, EOT, HEADER_SEP = 128000, 128006, 128007, 128009, 271


def gpt2_byte_table() -> list[str]:
    """Tokenizer::build_gpt2_byte_table, tokenizer.rs:56-75."""
    bs = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    cs = list(bs)
    n = 0
    for b in range(256):
        if b not in bs:
            bs.append(b)
            cs.append(256 + n)
            n += 1
    table = [""] * 256
    for b, c in zip(bs, cs):
        table[b] = chr(c)
    return table


def gpt2_split(text: str) -> list[str]:
    return GPT2_PATTERN.findall(text)


class OracleTokenizer:
    """Tokenizer::from_gguf_parts (tokenizer.rs:77-137) and its methods."""

    def __init__(self, vocab, merges, bos, eos, pre="default", add_bos_token=True, add_space_prefix=False,
                 chat_template=None, byte_level=True, scores=None):
        self.vocab = list(vocab)
        self.bos, self.eos, self.pre = bos, eos, pre
        self.add_bos_token, self.add_space_prefix = add_bos_token, add_space_prefix
        self.chat_template = chat_template
        self.byte_level = byte_level
        # HashMap collect: the last id of equal texts; binary_search on the
        # stable-sorted vocabulary lands on the same (last) entry
        self.index = {t: i for i, t in enumerate(self.vocab)}
        if scores is not None:
            self.scores = [float(np.float32(x)) for x in scores]
        else:
            self.scores = [0.0] * len(self.vocab)
            for i, m in enumerate(merges):
                parts = m.split(" ", 1)
                if len(parts) == 2:
                    j = self.index.get(parts[0] + parts[1])
                    if j is not None:
                        self.scores[j] = float(np.float32(len(merges) - i))
        if not byte_level:   # Tokenizer::new: byte b is token b + 3 (tokenizer.rs:259)
            self.char_to_byte, self.token_to_byte = {}, {}
            self.byte_to_token = [b + 3 for b in range(256)]
            return
        table = gpt2_byte_table()
        self.char_to_byte = {c: b for b, c in enumerate(table)}
        self.byte_to_token = [0] * 256
        self.token_to_byte = {}
        for b in range(256):
            j = self.index.get(table[b])
            if j is not None:
                self.byte_to_token[b] = j
                self.token_to_byte[j] = b

    @classmethod
    def from_hf_json(cls, path):
        """Tokenizer::from_json (tokenizer.rs:134-224): ids 0..=max id, gaps
        empty, added tokens over the vocabulary, string merges, bos/eos from
        the added tokens' names (defaults 128000 / 128009)."""
        with open(path, encoding="utf-8") as f:
            root = json.load(f)
        vocab_obj, added = root["model"]["vocab"], root["added_tokens"]
        max_id = max([v for v in vocab_obj.values()] + [t["id"] for t in added] + [0])
        vocab = [""] * (max_id + 1)
        for text, i in vocab_obj.items():
            vocab[i] = text
        for t in added:
            vocab[t["id"]] = t["content"]
        bos, eos = 128000, 128009
        for t in added:
            if t["content"] == "<|begin_of_text|>":
                bos = t["id"]
            if t["content"] in ("<|end_of_text|>", "<|eot_id|>"):
                eos = t["id"]
        return cls(vocab, root["model"]["merges"], bos, eos)

    @classmethod
    def from_llama2c(cls, path):
        """Tokenizer::new (tokenizer.rs:226-268): the llama2.c tokenizer.bin."""
        raw = open(path, "rb").read()
        n, _, bos, eos = struct.unpack_from("<4I", raw, 0)
        vocab, scores, o = [], [], 16
        for _ in range(n):
            sc, ln = struct.unpack_from("<fI", raw, o)
            o += 8
            vocab.append(raw[o:o + ln].decode("utf-8"))
            scores.append(sc)
            o += ln
        return cls(vocab, [], bos, eos, byte_level=False, scores=scores)

    def has_llama_tokens(self):
        return len(self.vocab) > 128009

    def bpe_merge(self, tokens):
        """tokenizer.rs:296-323: merge the adjacent pair whose concatenation
        is in the vocabulary with the highest score (first such pair on ties)."""
        while True:
            best_score, best_id, best_idx = -1e10, 0, -1
            for idx in range(len(tokens) - 1):
                j = self.index.get(self.vocab[tokens[idx]] + self.vocab[tokens[idx + 1]])
                if j is not None and self.scores[j] > best_score:
                    best_score, best_id, best_idx = self.scores[j], j, idx
            if best_idx == -1:
                return tokens
            tokens[best_idx] = best_id
            del tokens[best_idx + 1]

    def encode(self, text, bos=False, eos=False):
        """tokenizer.rs:325-380."""
        assert text, "Text to encode should not be empty"
        tokens = [self.bos] if bos else []
        if self.pre in ("gpt2", "smollm"):
            if self.add_space_prefix and not text.startswith(" "):
                text = " " + text
            for seg in gpt2_split(text):
                tokens += self.bpe_merge([self.byte_to_token[b] for b in seg.encode()])
        elif self.byte_level:
            tokens += [self.byte_to_token[b] for b in text.encode()]
            tokens = self.bpe_merge(tokens)
        else:
            for c in text:   # tokenizer.rs:356-370
                j = self.index.get(c)
                tokens += [j] if j is not None else [b + 3 for b in c.encode()]
            tokens = self.bpe_merge(tokens)
        if eos:
            tokens.append(self.eos)
        return tokens

    def decode(self, ids):
        """tokenizer.rs:540-568: byte-level ids through String::from_utf8_lossy,
        else the vocabulary texts concatenated."""
        if not self.byte_level:
            return "".join(self.vocab[t] for t in ids if t < len(self.vocab))
        out = bytearray()
        for t in ids:
            if t in self.token_to_byte:
                out.append(self.token_to_byte[t])
            elif t < len(self.vocab):
                for c in self.vocab[t]:
                    out += bytes([self.char_to_byte[c]]) if c in self.char_to_byte else c.encode()
        return out.decode("utf-8", errors="replace")

    def encode_wrap_n_header(self, text, header, wrap):
        """tokenizer.rs:243-286."""
        if not self.has_llama_tokens():
            toks = [self.bos] if wrap and self.add_bos_token else []
            return toks + (self.encode(text) if text else [])
        toks = [BEGIN_OF_TEXT] if wrap else []
        if header:
            toks += [START_HEADER] + self.encode(header) + [END_HEADER, HEADER_SEP]
        if text:
            toks += self.encode(text)
        if wrap:
            toks += [HEADER_SEP, EOT]
        return toks

    def render_chat_template(self, messages, add_generation_prompt):
        """tokenizer.rs:391-422 (minijinja there, jinja2 here)."""
        env = jinja2.Environment(keep_trailing_newline=False, autoescape=False)
        out = env.from_string(self.chat_template).render(
            messages=[{"role": r, "content": c} for r, c in messages], add_generation_prompt=add_generation_prompt)
        return self.encode_template_output(out) if out else []

    def encode_template_output(self, text):
        """tokenizer.rs:424-456: longest vocabulary text containing '<' at each '<'."""
        specials = {t: i for i, t in enumerate(self.vocab) if "<" in t}
        b = text.encode()
        sb = {t.encode(): i for t, i in specials.items()}
        out, pos = [], 0
        while pos < len(b):
            if b[pos:pos + 1] == b"<":
                best = max((k for k in sb if b.startswith(k, pos)), key=len, default=None)
                if best is not None:
                    out.append(sb[best])
                    pos += len(best)
                    continue
            start = pos
            pos += 1
            while pos < len(b) and b[pos:pos + 1] != b"<":
                pos += 1
            out += self.encode(b[start:pos].decode())
        return out

    def apply_system_template(self, system):
        """tokenizer.rs:496-514."""
        if self.chat_template is not None:
            return self.render_chat_template([("system", system)], False)
        if self.has_llama_tokens():
            return self.encode_wrap_n_header(system, "system", True)
        return self.encode(system) if system else []

    def apply_turn_template(self, user, add_empty_assistant):
        """tokenizer.rs:516-543."""
        if self.chat_template is not None:
            msgs = [("user", user)] + ([("assistant", "")] if add_empty_assistant else [])
            r = self.render_chat_template(msgs, add_empty_assistant)
            if add_empty_assistant and r and r[-1] == EOT:
                r.pop()
            return r
        if self.has_llama_tokens():
            u, a = self.encode("user"), self.encode("assistant")
            assert len(u) == 1 and len(a) == 1
            toks = [START_HEADER, u[0], END_HEADER, HEADER_SEP] + self.encode_wrap_n_header(user, "", False) + [EOT]
            if add_empty_assistant:
                toks += [START_HEADER, a[0], END_HEADER, HEADER_SEP]
            return toks
        return ([self.bos] if self.add_bos_token else []) + self.encode(user)

    def chat_prompt(self, user):
        """main.rs:148-152,183: the first turn's prompt."""
        if self.chat_template is None:
            pre = self.apply_system_template("")
        else:
            pre = [self.bos] if self.add_bos_token else []
        return pre + self.apply_turn_template(user.strip(RUST_WHITE_SPACE), True)


# str::trim's White_Space set
RUST_WHITE_SPACE = "".join(chr(c) for c in list(range(9, 14)) + [0x20, 0x85, 0xA0, 0x1680] + list(range(0x2000, 0x200B))
                           + [0x2028, 0x2029, 0x202F, 0x205F, 0x3000])

_libm = ctypes.CDLL("libm.so.6")
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]


def random_f32(seed: int) -> np.float32:
    """Sampler::random_u32 / random_f32 (sampler.rs:81-91): one xorshift64* step."""
    m = (1 << 64) - 1
    s = seed & m
    s ^= s >> 12
    s ^= (s << 25) & m
    s ^= s >> 27
    r = ((s * 0x2545F4914F6CDD1D) & m) >> 32
    return np.float32(np.float32(r >> 8) / np.float32(16777216.0))


class OracleSampler:
    """Sampler (sampler.rs:40-180)."""

    def __init__(self, vocab, temperature, top_p, seed):
        self.vocab = vocab
        self.temperature, self.top_p, self.seed = np.float32(temperature), np.float32(top_p), seed
        self.prob_idx = [(np.float32(0.0), 0)] * vocab   # persists across calls

    def sample(self, logits: np.ndarray) -> int:
        x = np.array(logits, np.float32)
        if self.temperature == 0:
            return _argmax_first(x)
        x = x / self.temperature
        mx = np.float32(-np.inf)
        for v in x:
            mx = np.fmax(mx, v)
        e = np.array([_libm.expf(float(np.float32(v - mx))) for v in x], np.float32)
        s = np.add.accumulate(e, dtype=np.float32)[-1]
        p = e / s
        rand = random_f32(self.seed)
        if self.top_p <= 0 or self.top_p >= 1:
            cdf = np.add.accumulate(p, dtype=np.float32)
            for i, c in enumerate(cdf):
                if rand < c:
                    return i
            return len(p) - 1
        n = len(p)
        cutoff = np.float32(np.float32(1.0) - self.top_p) / np.float32(n - 1)
        n0 = 0
        arr = list(self.prob_idx)
        for i, v in enumerate(p):
            if v >= cutoff:
                arr[n0] = (v, i)
                n0 += 1
        arr = sorted(arr, key=lambda t: -float(t[0]))   # stable, descending
        self.prob_idx = arr
        cum = np.float32(0.0)
        last = n0 - 1
        for i in range(n0):
            cum = np.float32(cum + arr[i][0])
            if cum > self.top_p:
                last = i
                break
        r = np.float32(rand * cum)
        cdf = np.float32(0.0)
        for i in range(last + 1):
            cdf = np.float32(cdf + arr[i][0])
            if r < cdf:
                return arr[i][1]
        return arr[last][1]


def _argmax_first(x) -> int:
    """Sampler::sample_argmax (sampler.rs:67-79)."""
    mi, mp = 0, x[0]
    for i in range(1, len(x)):
        if x[i] > mp:
            mi, mp = i, x[i]
    return mi
