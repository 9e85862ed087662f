"""Tokenizer and Sampler over the library's host-side C++ implementation.

Python mirror of the reference's tokenizer.rs and sampler.rs:
  Tokenizer.encode / decode            tokenizer.rs:325-380, 545-568
  Tokenizer.encode_wrap_n_header       tokenizer.rs:243-286
  Tokenizer.apply_system_template      tokenizer.rs:496-514
  Tokenizer.apply_turn_template        tokenizer.rs:516-543 (chat template
                                       rendered as minijinja renders it)
  Sampler(vocab, temperature, top_p, seed).sample(logits)
                                       sampler.rs:40-180
A Tokenizer comes from a GGUF file's metadata (Tokenizer.from_gguf, no GPU
needed) or from a loaded model (Transformer.tokenizer()).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from ._lib import YlError, check, last_error, lib


def _ids(fn, *args) -> list[int]:
    n = C.c_size_t(0)
    cap = 256
    while True:
        buf = np.zeros(cap, np.uint32)
        st = fn(*args, buf.ctypes.data, cap, C.byref(n))
        if st == -8 and n.value > cap:   # YL_ERR_RANGE: grow to the reported length
            cap = n.value
            continue
        check(st)
        return [int(x) for x in buf[:n.value]]


class Tokenizer:
    """tokenizer.rs Tokenizer, built from GGUF tokenizer metadata."""

    def __init__(self, handle, owner=None):
        self._h = handle
        self._owner = owner   # the model that owns the handle, or None (owned here)

    @classmethod
    def from_file(cls, path: str) -> "Tokenizer":
        """tokenizer.json (Tokenizer::from_json), tokenizer.bin
        (Tokenizer::new) or a GGUF file (Tokenizer::from_gguf_parts), by the
        file's extension."""
        h = lib().yl_tokenizer_load(os.fsencode(path))
        if not h:
            raise YlError(-4, last_error())
        return cls(h)

    from_gguf = from_file
    from_json = from_file

    @property
    def vocab_size(self) -> int:
        return int(lib().yl_tokenizer_vocab_size(self._h))

    def encode(self, text: str, bos: bool = False, eos: bool = False) -> list[int]:
        return _ids(lib().yl_tokenize, self._h, text.encode(), int(bos), int(eos))

    def decode(self, token_ids) -> str:
        t = np.ascontiguousarray(token_ids, np.uint32)
        n = C.c_size_t(0)
        st = lib().yl_detokenize(self._h, t.ctypes.data, t.size, None, 0, C.byref(n))
        if st not in (0, -8):
            check(st)
        buf = C.create_string_buffer(n.value + 1)
        check(lib().yl_detokenize(self._h, t.ctypes.data, t.size, buf, n.value + 1, C.byref(n)))
        return buf.raw[:n.value].decode()

    def apply_system_template(self, system: str) -> list[int]:
        return _ids(lib().yl_chat_template, self._h, 0, system.encode(), 0)

    def apply_turn_template(self, user: str, add_empty_assistant: bool) -> list[int]:
        return _ids(lib().yl_chat_template, self._h, 1, user.encode(), int(add_empty_assistant))

    def encode_wrap_n_header(self, text: str, begin_of_text_wrap: bool) -> list[int]:
        """encode_wrap_n_header(text, "", begin_of_text_wrap)."""
        return _ids(lib().yl_chat_template, self._h, 2, text.encode(), int(begin_of_text_wrap))

    def chat_prompt(self, user: str) -> list[int]:
        """The CLI's first-turn prompt (main.rs:148-152,183)."""
        return _ids(lib().yl_chat_prompt, self._h, user.encode())

    def close(self) -> None:
        if self._h and self._owner is None:
            lib().yl_tokenizer_free(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def pretokenize(text: str) -> list[str]:
    """The GPT-2 pre-tokenizer split (tokenizer.rs:29-31) as the library runs it."""
    raw = text.encode()
    b = _ids(lib().yl_pretokenize, raw)
    return [raw[b[k]:b[k + 1]].decode() for k in range(0, len(b), 2)]


class Sampler:
    """sampler.rs Sampler: argmax at temperature 0, else softmax(logits /
    temperature) and multinomial or top-p sampling from a fixed draw."""

    def __init__(self, vocab_size: int, temperature: float, top_p: float, seed: int):
        self.vocab_size = vocab_size
        self._h = lib().yl_sampler_new(vocab_size, temperature, top_p, seed)
        if not self._h:
            raise YlError(-1, last_error())

    def sample(self, logits: np.ndarray) -> int:
        """Samples a token; like the reference, rewrites `logits` (f32, in place)."""
        if logits.dtype != np.float32 or not logits.flags.c_contiguous or logits.size != self.vocab_size:
            raise ValueError("logits must be a contiguous float32 array of vocab_size")
        out = C.c_uint32(0)
        check(lib().yl_sampler_sample(self._h, logits.ctypes.data, C.byref(out)))
        return int(out.value)

    def close(self) -> None:
        if self._h:
            lib().yl_sampler_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
