"""Byte-level BPE vocabularies for the tokenizer tests (test infrastructure).

A vocabulary is trained with the Hugging Face `tokenizers` library on a small
built-in corpus, giving the GGUF-style token strings (GPT-2 byte characters)
and "left right" merges that llama.cpp writes into tokenizer.ggml.tokens and
tokenizer.ggml.merges.
"""
from __future__ import annotations

import json

CORPUS = [
    "The quick brown fox jumps over the lazy dog. The dog sleeps; the fox runs away!",
    "user assistant user assistant system user assistant",
    "Hello, world! Hello again, world. It's a small world, isn't it? We'll see, we've seen, they're here.",
    "Numbers: 0 1 2 3 42 1234 2024 3.14159 -17 +8 100% 7/8",
    "Mixed   spacing\tand\ttabs\nnew lines\n\nand more  text   here",
    "Unicode: über café naïve résumé — “quotes” ‘single’ © ® ™ € £ ¥",
    "中文 文本 测试 日本語 テキスト 한국어 텍스트 Ελληνικά русский текст العربية עברית",
    "emoji 😀 🚀 🌍 and symbols ★ ☆ ✓ ✗ → ← ↑ ↓",
    "code: def f(x): return x**2 if x > 0 else -x  # comment",
    "<|im_start|>user hi<|im_end|> <|im_start|>assistant hello<|im_end|>",
    "She said: 'I'm sure you'd like it, I'd think.' He replied: 'You'll love it.'",
    "Lorem ipsum dolor sit amet, consectetur adipiscing elit, sed do eiusmod tempor incididunt ut labore.",
] * 8

SPECIALS = ["<|bos|>", "<|eos|>", "<|im_start|>", "<|im_end|>"]


def train(vocab_size: int = 700):
    """Returns (tokens list ordered by id, merges list)."""
    from tokenizers import Tokenizer, models, pre_tokenizers, trainers

    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    trainer = trainers.BpeTrainer(vocab_size=vocab_size, initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                                  special_tokens=SPECIALS, show_progress=False)
    tok.train_from_iterator(CORPUS, trainer)
    model = json.loads(tok.to_str())["model"]
    vocab = model["vocab"]
    tokens = [None] * len(vocab)
    for t, i in vocab.items():
        tokens[i] = t
    merges = [m if isinstance(m, str) else " ".join(m) for m in model["merges"]]
    return tokens, merges, tok


def hf_bpe_segment(hf_tokenizer, mapped: str) -> list[int]:
    """The Hugging Face BPE model alone on one pre-split, byte-mapped piece."""
    return [t.id for t in hf_tokenizer.model.tokenize(mapped)]
