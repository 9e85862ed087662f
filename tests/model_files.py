"""Synthetic safetensors and lm.rs model directories for the loader tests
(test infrastructure): the package's writers (synth_files) with a trained
byte-level BPE vocabulary as tokenizer.json, or the llama2.c tokenizer.bin.
"""
from __future__ import annotations

import json
import os

import bpe_vocab
from yallma3_mini_inference_amd.synth_files import Shape, llama2c_tokenizer_bin, write_lmrs  # noqa: F401
from yallma3_mini_inference_amd import synth_files as SF


def hf_tokenizer_json(path: str):
    """A trained byte-level BPE vocabulary as tokenizer.json, with
    <|begin_of_text|> / <|eot_id|> added after a gap of two unused ids.
    Returns the vocabulary size (max id + 1)."""
    tokens, merges, _ = bpe_vocab.train()
    vocab = {t: i for i, t in enumerate(tokens)}
    n = len(tokens)
    added = [{"id": i, "content": t, "special": True} for i, t in enumerate(bpe_vocab.SPECIALS)]
    added += [{"id": n + 2, "content": "<|begin_of_text|>", "special": True},
              {"id": n + 3, "content": "<|eot_id|>", "special": True}]
    root = {"version": "1.0", "added_tokens": added,
            "model": {"type": "BPE", "vocab": vocab, "merges": merges}}
    with open(path, "w", encoding="utf-8") as f:
        json.dump(root, f, ensure_ascii=False)
    return n + 4


def write_safetensors(d: str, s: Shape, vocab: int | None = None, q8_gs: int = 0, seed: int = 0,
                      tokenizer: str = "json") -> str:
    """SF.write_safetensors with the trained tokenizer.json ("json") or the
    llama2.c tokenizer.bin ("bin")."""
    if tokenizer == "json":
        tok = lambda dd: hf_tokenizer_json(os.path.join(dd, "tokenizer.json"))
    else:
        tok = lambda dd: len(llama2c_tokenizer_bin(os.path.join(dd, "tokenizer.bin"))[0])
    return SF.write_safetensors(d, s, vocab=vocab, q8_gs=q8_gs, seed=seed, tokenizer=tok)
