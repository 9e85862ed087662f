"""CPU restatement of the reference's safetensors and lm.rs model loaders.

TEST INFRASTRUCTURE ONLY (imported by tests/, never by the product package).
Parses the files with Python's json module and numpy (no code shared with the
library's C++ loaders) and builds an oracle Model (oracle.Model.from_arrays)
whose forward pass is the C oracle's, with util::rope (HF layout) and the
file's group size.  Tokenizers come from oracle/tokenizer.py.
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np

from . import oracle as O
from . import tokenizer as OT


# binary16 -> float32 for every bit pattern (numpy's IEEE conversion), used as
# a lookup table: numpy converts half floats one element at a time.
_F16_TO_F32 = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)


def _f16(raw: bytes, count: int, offset: int) -> np.ndarray:
    return _F16_TO_F32[np.frombuffer(raw, np.uint16, count, offset)]


def _round_away(x: np.ndarray) -> np.ndarray:
    """Rust f32::round (half away from zero), exactly (in float64)."""
    x = x.astype(np.float64)
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def load_q8_tensor_st(raw: bytes, rows: int, cols: int, gs: int, w_off: int, s_off: int, b_off: int):
    """util::load_q8_tensor_st (util.rs:452-503): u8 * f16 scale + f16 bias per
    group, requantized symmetric (scale = max|v| / 127, or 1 for an all-zero
    group), values round-half-away and clamped to [-128, 127]."""
    n = rows * cols
    groups = n // gs
    vals = np.frombuffer(raw, np.uint8, n, w_off).astype(np.float32)
    scale = _f16(raw, groups, s_off)
    bias = _f16(raw, groups, b_off)
    deq = (vals.reshape(groups, gs) * scale[:, None]).astype(np.float32) + bias[:, None]
    deq = deq.astype(np.float32)
    max_abs = np.max(np.abs(deq), axis=1)
    sym = np.where(max_abs == 0, np.float32(1.0), (max_abs / np.float32(127.0)).astype(np.float32)).astype(np.float32)
    q = np.clip(_round_away((deq / sym[:, None]).astype(np.float32)), -128, 127).astype(np.int8)
    return q.ravel(), sym


def _tokenizer_beside(model_dir: str):
    tj = os.path.join(model_dir, "tokenizer.json")
    if os.path.exists(tj):
        return OT.OracleTokenizer.from_hf_json(tj)
    return OT.OracleTokenizer.from_llama2c(os.path.join(model_dir, "tokenizer.bin"))


def read_safetensors(path: str, max_ctx_len: int = 0xFFFFFFFF) -> dict:
    """TransformerLlamaSt::load_model_inner (transformer_llama_st.rs:41-300)
    as arrays: shape, eps, rope_theta, gs, fmt, embedding (f32), norms and
    layers[l] = 7 projections (q, k, v, o, gate, down, up)."""
    d = os.path.dirname(path)
    with open(os.path.join(d, "config.json")) as f:
        cfg = json.load(f)
    dim, hidden = cfg["hidden_size"], cfg["intermediate_size"]
    nh, nkv, hd = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    nl, vocab = cfg["num_hidden_layers"], cfg["vocab_size"]
    eps, theta = float(np.float32(cfg["rms_norm_eps"])), float(np.float32(cfg["rope_theta"]))
    ctx = min(cfg["max_position_embeddings"], max_ctx_len)
    q = cfg.get("quantization")
    f16 = q is None
    gs = 32 if f16 else q.get("group_size", 32)
    raw = open(path, "rb").read()
    hlen = struct.unpack_from("<Q", raw, 0)[0]
    hdr = json.loads(raw[8:8 + hlen])
    start = 8 + hlen
    off = {k: start + v["data_offsets"][0] for k, v in hdr.items() if k != "__metadata__"}
    f16v = lambda name, n: _f16(raw, n, off[name])
    out = {"shape": (dim, hidden, nl, nh, nkv, hd, vocab, ctx), "eps": eps, "rope_theta": theta, "gs": gs,
           "fmt": O.F16 if f16 else O.Q8_0}
    out["rms_final"] = f16v("model.norm.weight", dim)
    out["rms_att"] = [f16v(f"model.layers.{l}.input_layernorm.weight", dim) for l in range(nl)]
    out["rms_ffn"] = [f16v(f"model.layers.{l}.post_attention_layernorm.weight", dim) for l in range(nl)]
    if f16:
        out["embedding"] = f16v("model.embed_tokens.weight", vocab * dim)
    else:
        qv, sc = load_q8_tensor_st(raw, vocab, dim, gs, off["model.embed_tokens.weight"],
                                   off["model.embed_tokens.scales"], off["model.embed_tokens.biases"])
        out["embedding"] = (qv.astype(np.float32) * np.repeat(sc, gs)).astype(np.float32)
    names = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
             "mlp.down_proj", "mlp.up_proj"]
    qr, kr = nh * hd, nkv * hd
    shapes = [(qr, dim), (kr, dim), (kr, dim), (dim, qr), (hidden, dim), (dim, hidden), (hidden, dim)]
    layers = []
    for l in range(nl):
        projs = []
        for nm, (r, c) in zip(names, shapes):
            base = f"model.layers.{l}.{nm}"
            if f16:
                projs.append(f16v(base + ".weight", r * c))
            else:
                projs.append(load_q8_tensor_st(raw, r, c, gs, off[base + ".weight"], off[base + ".scales"],
                                               off[base + ".biases"]))
        layers.append(projs)
    out["layers"] = layers
    return out


def _model(a: dict):
    return O.Model.from_arrays(a["shape"], a["eps"], a["rope_theta"], a["gs"], True, a["fmt"], a["embedding"],
                               a["rms_final"], a["rms_att"], a["rms_ffn"], a["layers"])


def load_safetensors(path: str, max_ctx_len: int = 0xFFFFFFFF):
    """The oracle model and tokenizer of a safetensors directory."""
    return _model(read_safetensors(path, max_ctx_len)), _tokenizer_beside(os.path.dirname(path))


def read_lmrs(path: str, max_ctx_len: int = 0xFFFFFFFF) -> dict:
    """TransformerLlamaLmrs::load_model_inner (transformer_llama_lmrs.rs:60-434)
    as arrays (the keys of read_safetensors)."""
    raw = open(path, "rb").read()
    assert raw[:4] == b"lmrs", "Model not in lm.rs format."
    (dim, hidden, nl, nh, hs, nkv, vocab, seq_len) = struct.unpack_from("<8I", raw, 8)
    eps, theta = struct.unpack_from("<2f", raw, 40)
    gs = struct.unpack_from("<I", raw, 50)[0]
    ctx = min(seq_len, max_ctx_len)
    pos = [256]

    def q8(count):
        g = count // gs
        qv = np.frombuffer(raw, np.int8, count, pos[0])
        sc = np.frombuffer(raw, np.float32, g, pos[0] + count)
        pos[0] += count + 4 * g
        return qv, sc

    def f32(count):
        v = np.frombuffer(raw, np.float32, count, pos[0])
        pos[0] += 4 * count
        return v

    eq, es = q8(vocab * dim)
    out = {"shape": (dim, hidden, nl, nh, nkv, hs, vocab, ctx), "eps": float(eps), "rope_theta": float(theta),
           "gs": gs, "fmt": O.Q8_0}
    out["embedding"] = (eq.astype(np.float32) * np.repeat(es, gs)).astype(np.float32)
    out["rms_att"] = [f32(dim) for _ in range(nl)]
    att, kv = nh * hs, nkv * hs
    wq = [q8(att * dim) for _ in range(nl)]
    wk = [q8(kv * dim) for _ in range(nl)]
    wv = [q8(kv * dim) for _ in range(nl)]
    wo = [q8(att * dim) for _ in range(nl)]
    out["rms_ffn"] = [f32(dim) for _ in range(nl)]
    w1 = [q8(hidden * dim) for _ in range(nl)]
    w2 = [q8(hidden * dim) for _ in range(nl)]
    w3 = [q8(hidden * dim) for _ in range(nl)]
    out["rms_final"] = f32(dim)
    out["layers"] = [[wq[l], wk[l], wv[l], wo[l], w1[l], w2[l], w3[l]] for l in range(nl)]
    out["end"] = pos[0]
    return out


def load_lmrs(path: str, max_ctx_len: int = 0xFFFFFFFF):
    """The oracle model and tokenizer of an lm.rs file (tokenizer.bin beside it)."""
    return (_model(read_lmrs(path, max_ctx_len)),
            OT.OracleTokenizer.from_llama2c(os.path.join(os.path.dirname(path), "tokenizer.bin")))
