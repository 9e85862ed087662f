"""Synthetic lm.rs and safetensors model directories (seeded random weights).

A safetensors directory holds config.json, model.safetensors and a
tokenizer.json (or tokenizer.bin): the layout TransformerLlamaSt reads
(transformer_llama_st.rs:41-300), with F16 tensors, or MLX-style 8-bit affine
groups (u8 values packed four to a U32, F16 scales and biases per group,
quantization.group_size in config.json).  An lm.rs directory holds
model.lmrs (the "lmrs" magic, the packed TransformerArgs at bytes 8..55,
weights from byte 256: transformer_llama_lmrs.rs:31-47, :150-434) and a
llama2.c tokenizer.bin (tokenizer.rs:226-268).

Weights are random (numpy's PCG64 with the given seed): projections scaled
by 1/sqrt(input width), norm weights near 1.  They exercise the loaders and
the forward pass at a real shape; they are not a trained model.
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass

import numpy as np


@dataclass
class Shape:
    dim: int = 128
    hidden: int = 256
    n_layers: int = 2
    n_heads: int = 4
    n_kv: int = 2
    head_dim: int = 32
    ctx: int = 256
    eps: float = 1e-5
    rope_theta: float = 500000.0


# Llama-3.2-1B: dim 2048, FFN 8192, 16 layers, 32 query / 8 KV heads of 64,
# vocabulary 128256 (the tokenizer is padded to it), context capped at 4096.
LLAMA32_1B = Shape(2048, 8192, 16, 32, 8, 64, 4096, 1e-5, 500000.0)
LLAMA32_1B_VOCAB = 128256


# ----------------------------------------------------------------- tokenizers
LLAMA2C_PIECES = ["th", "he", "the", " t", " the", "in", "an", "and", " a", " an", " and", "er", "re", "on", "ou",
                  "is", "it", "at", "en", "es", "or", "ing", " i", " in", " is", " it", "qu", "ick", "row", "own",
                  " b", " br", " brown", "fo", "ox", " f", " fox", "lo", "ll", "llo", "ello", "He", "Hello", " w",
                  "or", "orl", "orld", " world", "um", "ps", "mp", "ju", " j", " jump", " jumps", "az", "zy", " l",
                  " lazy", "do", "og", " d", " dog", "é", "ca", "caf", "café", " über", "ü", "be", "ber", "über"]


def llama2c_tokenizer_bin(path: str, n_pad: int = 0, vocab: int | None = None):
    """A llama2.c tokenizer.bin: <unk> <s> </s>, the 256 byte pieces
    <0x00>..<0xFF> (ids 3..258), the printable ASCII characters, then merged
    pieces with falling scores (two share a score, so ties are exercised),
    then unused pieces (n_pad of them, or up to `vocab` entries).  Returns
    (pieces, scores, bos, eos)."""
    pieces = ["<unk>", "<s>", "</s>"] + [f"<0x{b:02X}>" for b in range(256)]
    scores = [0.0, 0.0, 0.0] + [0.0] * 256
    for c in range(32, 127):
        pieces.append(chr(c))
        scores.append(-1000.0 - c)
    seen = set(pieces)
    k = 0
    for p in LLAMA2C_PIECES:
        if p in seen:
            continue
        seen.add(p)
        pieces.append(p)
        scores.append(-float(k // 2 * 2) if k < 6 else -float(k))
        k += 1
    if vocab is not None:
        n_pad = max(0, vocab - len(pieces))
    for i in range(n_pad):
        pieces.append(f"<pad{i}>")
        scores.append(-1e6)
    bos, eos = 1, 2
    with open(path, "wb") as f:
        f.write(struct.pack("<4I", len(pieces), max(len(p.encode()) for p in pieces), bos, eos))
        for p, sc in zip(pieces, scores):
            b = p.encode()
            f.write(struct.pack("<fI", sc, len(b)))
            f.write(b)
    return pieces, scores, bos, eos


def gpt2_byte_chars() -> list[str]:
    """The byte -> character table of byte-level BPE (tokenizer.rs:40-61)."""
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


def byte_tokenizer_json(path: str, vocab: int | None = None) -> int:
    """A byte-level tokenizer.json without training: the 256 byte characters,
    merges of LLAMA2C_PIECES built left to right, unused entries up to
    `vocab`, and <|begin_of_text|> / <|eot_id|> as the last two ids.
    Returns the vocabulary size (max id + 1)."""
    table = gpt2_byte_chars()
    tokens = list(table)
    index = {t: i for i, t in enumerate(tokens)}
    merges = []
    for piece in LLAMA2C_PIECES:
        mapped = "".join(table[b] for b in piece.encode())
        cur = mapped[0]
        for ch in mapped[1:]:
            nxt = cur + ch
            if nxt not in index:
                index[nxt] = len(tokens)
                tokens.append(nxt)
                merges.append(f"{cur} {ch}")
            cur = nxt
    total = max(vocab or 0, len(tokens) + 2)
    for i in range(len(tokens), total - 2):
        tokens.append(f"<unused{i}>")
    bos, eot = total - 2, total - 1
    root = {"version": "1.0",
            "added_tokens": [{"id": bos, "content": "<|begin_of_text|>", "special": True},
                             {"id": eot, "content": "<|eot_id|>", "special": True}],
            "model": {"type": "BPE", "vocab": {t: i for i, t in enumerate(tokens)}, "merges": merges}}
    with open(path, "w", encoding="utf-8") as f:
        json.dump(root, f, ensure_ascii=False)
    return total


# ----------------------------------------------------------------- weights
def _proj_shapes(s: Shape):
    q, kv = s.n_heads * s.head_dim, s.n_kv * s.head_dim
    return {"self_attn.q_proj": (q, s.dim), "self_attn.k_proj": (kv, s.dim), "self_attn.v_proj": (kv, s.dim),
            "self_attn.o_proj": (s.dim, q), "mlp.gate_proj": (s.hidden, s.dim), "mlp.down_proj": (s.dim, s.hidden),
            "mlp.up_proj": (s.hidden, s.dim)}


def _st_write(path, tensors):
    """safetensors: u64 header length, JSON header, data (8-byte aligned)."""
    hdr, off = {"__metadata__": {"format": "mlx"}}, 0
    for name, (dtype, shape, data) in tensors.items():
        hdr[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + data.nbytes]}
        off += data.nbytes
    h = json.dumps(hdr).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for _, (_, _, data) in tensors.items():
            f.write(np.ascontiguousarray(data).tobytes())


def write_safetensors(d: str, s: Shape, vocab: int | None = None, q8_gs: int = 0, seed: int = 0,
                      tokenizer=None) -> str:
    """model.safetensors + config.json + a tokenizer in directory d; F16 when
    q8_gs == 0, else 8-bit affine groups of q8_gs.  `tokenizer(d) -> size`
    writes the tokenizer (default: byte_tokenizer_json padded to `vocab`);
    the model's vocabulary is `vocab`, else the tokenizer's size.  Returns
    the model path."""
    os.makedirs(d, exist_ok=True)
    if tokenizer is None:
        v_tok = byte_tokenizer_json(os.path.join(d, "tokenizer.json"), vocab)
    else:
        v_tok = tokenizer(d)
    V = vocab or v_tok
    r = np.random.default_rng(seed)
    cfg = {"architectures": ["LlamaForCausalLM"], "hidden_size": s.dim, "intermediate_size": s.hidden,
           "num_attention_heads": s.n_heads, "num_key_value_heads": s.n_kv, "head_dim": s.head_dim,
           "num_hidden_layers": s.n_layers, "vocab_size": V, "rms_norm_eps": s.eps, "rope_theta": s.rope_theta,
           "max_position_embeddings": s.ctx}
    if q8_gs:
        cfg["quantization"] = {"group_size": q8_gs, "bits": 8}
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(cfg, f)
    t = {}

    def f16(name, shape, scale, center=0.0):
        # uniform over 4096 levels with standard deviation `scale` (a lookup
        # table: numpy converts to binary16 one element at a time)
        levels = (center + (np.arange(-2048, 2048, dtype=np.float64) + 0.5) * (scale * np.sqrt(3.0) / 2048))
        t[name] = ("F16", shape, levels.astype(np.float16)[r.integers(0, 4096, size=shape, dtype=np.uint16)])

    def q8(base, rows, cols, scale):
        g = rows * cols // q8_gs
        vals = r.integers(0, 256, rows * cols, dtype=np.uint8)
        sc = (scale / 127.0 * (0.5 + r.random(g))).astype(np.float16)
        bias = (-(sc.astype(np.float32) * 128.0) * (0.8 + 0.4 * r.random(g))).astype(np.float16)
        if g > 2:   # an all-zero group (symmetric scale 1) and a one-sided one
            vals[:q8_gs] = 0
            sc[0], bias[0] = 0.0, 0.0
            bias[1] = np.float16(0.0)
        t[base + ".weight"] = ("U32", (rows, cols // 4), vals.view(np.uint32))
        t[base + ".scales"] = ("F16", (rows, cols // q8_gs), sc)
        t[base + ".biases"] = ("F16", (rows, cols // q8_gs), bias)

    if q8_gs:
        q8("model.embed_tokens", V, s.dim, 0.3)
    else:
        f16("model.embed_tokens.weight", (V, s.dim), 0.15)
    f16("model.norm.weight", (s.dim,), 0.1, 1.0)
    for l in range(s.n_layers):
        p = f"model.layers.{l}."
        f16(p + "input_layernorm.weight", (s.dim,), 0.1, 1.0)
        f16(p + "post_attention_layernorm.weight", (s.dim,), 0.1, 1.0)
        for nm, (rows, cols) in _proj_shapes(s).items():
            if q8_gs:
                q8(p + nm, rows, cols, 2.0 / np.sqrt(cols))
            else:
                f16(p + nm + ".weight", (rows, cols), 0.7 / np.sqrt(cols))
    path = os.path.join(d, "model.safetensors")
    _st_write(path, t)
    return path


def write_lmrs(d: str, s: Shape, gs: int = 32, seed: int = 0, n_pad: int = 0, vocab: int | None = None) -> str:
    """model.lmrs + tokenizer.bin (llama2c_tokenizer_bin) in directory d.
    Returns the model path."""
    os.makedirs(d, exist_ok=True)
    V = len(llama2c_tokenizer_bin(os.path.join(d, "tokenizer.bin"), n_pad, vocab)[0])
    r = np.random.default_rng(seed)
    head = bytearray(256)
    head[0:4] = b"lmrs"
    struct.pack_into("<I", head, 4, 1)
    struct.pack_into("<8I2fBBIB", head, 8, s.dim, s.hidden, s.n_layers, s.n_heads, s.head_dim, s.n_kv, V, s.ctx,
                     s.eps, s.rope_theta, 0, 0, gs, 0)
    path = os.path.join(d, "model.lmrs")
    with open(path, "wb") as f:
        f.write(bytes(head))

        def q8(rows, cols, scale):
            f.write(r.integers(-127, 128, rows * cols, dtype=np.int8).tobytes())
            f.write((scale / 127.0 * (0.5 + r.random(rows * cols // gs))).astype(np.float32).tobytes())

        def norm():
            f.write((1.0 + 0.1 * r.standard_normal(s.dim)).astype(np.float32).tobytes())

        q8(V, s.dim, 0.3)
        L = s.n_layers
        att, kv = s.n_heads * s.head_dim, s.n_kv * s.head_dim
        for _ in range(L):
            norm()
        for rows, cols in [(att, s.dim), (kv, s.dim), (kv, s.dim), (s.dim, att)]:
            for _ in range(L):
                q8(rows, cols, 2.0 / np.sqrt(cols))
        for _ in range(L):
            norm()
        for rows, cols in [(s.hidden, s.dim), (s.dim, s.hidden), (s.hidden, s.dim)]:
            for _ in range(L):
                q8(rows, cols, 2.0 / np.sqrt(cols))
        norm()
    return path


def ensure(name: str, root: str | None = None) -> str:
    """A cached Llama-3.2-1B-shaped model directory: "lmrs_1b" (lm.rs, Q8,
    group size 32), "st_q8_1b" (safetensors Q8, group size 64, the MLX 8-bit
    default) or "st_f16_1b" (safetensors, F16); returns the model path."""
    from .synth import model_dir
    d = os.path.join(root or model_dir(), name)
    if name == "lmrs_1b":
        path = os.path.join(d, "model.lmrs")
        if not os.path.exists(path):
            write_lmrs(d, LLAMA32_1B, gs=32, seed=11, vocab=LLAMA32_1B_VOCAB)
        return path
    if name == "st_q8_1b":
        path = os.path.join(d, "model.safetensors")
        if not os.path.exists(path):
            write_safetensors(d, LLAMA32_1B, vocab=LLAMA32_1B_VOCAB, q8_gs=64, seed=13)
        return path
    if name == "st_f16_1b":
        path = os.path.join(d, "model.safetensors")
        if not os.path.exists(path):
            write_safetensors(d, LLAMA32_1B, vocab=LLAMA32_1B_VOCAB, seed=12)
        return path
    raise KeyError(name)
