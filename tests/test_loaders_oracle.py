"""Pins of the oracle's safetensors / lm.rs restatement (CPU): util::rope
(HF layout, llama3 frequency scaling), util::load_q8_tensor_st, the two
file layouts, Tokenizer::from_json and Tokenizer::new (llama2.c) -- and the
library's tokenizer.json / tokenizer.bin tokenizers against the oracle."""
from __future__ import annotations

import json
import math
import struct

import numpy as np
import pytest

import bpe_vocab
import model_files as MF
from oracle import loaders as L
from oracle import oracle as O
from oracle import tokenizer as OT


# ----------------------------------------------------------------- util::rope
def _freq64(j, head, theta, ctx):
    """The llama3 frequency of pair j in float64 (the published scaling:
    factor 32, low 1, high 4, original context = ctx)."""
    f = theta ** (-(2 * j) / head)
    wl = 2 * math.pi / f
    if wl > ctx:
        return f / 32.0
    if wl >= ctx / 4.0:
        s = (ctx / wl - 1.0) / 3.0
        return (1 - s) * f / 32.0 + s * f
    return f


def test_rope_hf_position_zero_is_identity():
    r = np.random.default_rng(0)
    q = r.standard_normal(4 * 64).astype(np.float32)
    k = r.standard_normal(2 * 64).astype(np.float32)
    q0, k0 = q.copy(), k.copy()
    O.rope_hf(q, k, 64, 4, 2, 500000.0, 256, 0)
    assert np.array_equal(q, q0) and np.array_equal(k, k0)


@pytest.mark.parametrize("pos", [1, 3, 17])
def test_rope_hf_pairs_and_frequencies(pos):
    head, theta, ctx = 64, 500000.0, 256
    half = head // 2
    regimes = set()
    for j in range(half):
        f64 = _freq64(j, head, theta, ctx)
        wl = 2 * math.pi / (theta ** (-(2 * j) / head))
        regimes.add("high" if wl < ctx / 4 else "low" if wl > ctx else "mid")
        for head_idx in range(2):
            q = np.zeros(2 * head, np.float32)
            k = np.zeros(head, np.float32)
            q[head_idx * head + j] = 1.0          # (1, 0) in pair (j, j + half)
            k[j + half] = 1.0                      # (0, 1)
            O.rope_hf(q, k, head, 2, 1, theta, ctx, pos)
            nz = sorted(np.flatnonzero(q).tolist())
            assert set(nz) <= {head_idx * head + j, head_idx * head + j + half}
            ang = (pos * f64) % (2 * math.pi)
            c, s = q[head_idx * head + j], q[head_idx * head + j + half]
            assert abs(c - math.cos(ang)) < 2e-5 and abs(s - math.sin(ang)) < 2e-5
            assert abs(k[j] + math.sin(ang)) < 2e-5 and abs(k[j + half] - math.cos(ang)) < 2e-5
    assert regimes == {"high", "mid", "low"}


def test_rope_hf_preserves_pair_norms():
    r = np.random.default_rng(1)
    q = r.standard_normal(4 * 32).astype(np.float32)
    k = r.standard_normal(2 * 32).astype(np.float32)
    q0 = q.astype(np.float64).reshape(4, 2, 16)
    O.rope_hf(q, k, 32, 4, 2, 10000.0, 128, 77)
    q1 = q.astype(np.float64).reshape(4, 2, 16)
    assert np.allclose(np.hypot(q0[:, 0], q0[:, 1]), np.hypot(q1[:, 0], q1[:, 1]), rtol=1e-5)


# ------------------------------------------------------ load_q8_tensor_st
def _st_group(vals, scale, bias):
    raw = np.asarray(vals, np.uint8).tobytes() + np.float16(scale).tobytes() + np.float16(bias).tobytes()
    n = len(vals)
    return L.load_q8_tensor_st(raw, 1, n, n, 0, n, n + 2)


def test_load_q8_st_hand_worked_group():
    # u8 * 0.5 - 0.5: 255 -> 127 (the group's max, so the symmetric scale is
    # exactly 1), 6 -> 2.5 (half rounds away: 3), 0 -> -0.5 (-> -1), 1 -> 0
    vals = [255, 6, 0, 1] + [2] * 28
    q, s = _st_group(vals, 0.5, -0.5)
    assert s.tolist() == [1.0]
    assert q[:5].tolist() == [127, 3, -1, 0, 1]


def test_load_q8_st_zero_group_and_scale():
    q, s = _st_group([0] * 32, 0.0, 0.0)
    assert s.tolist() == [1.0] and not q.any()
    # a group of one value v: max |v| maps to +-127
    q, s = _st_group([10] * 32, 0.25, -5.0)     # 10 * 0.25 - 5 = -2.5
    assert s[0] == np.float32(2.5) / np.float32(127.0) and (q == -127).all()


def test_load_q8_st_requant_error_bound():
    r = np.random.default_rng(3)
    vals = r.integers(0, 256, 64, dtype=np.uint8)
    q, s = _st_group(vals, 0.013, -1.7)
    deq = vals.astype(np.float32) * np.float32(np.float16(0.013)) + np.float32(np.float16(-1.7))
    assert np.max(np.abs(q * s[0] - deq)) <= s[0] / 2 * 1.0001
    assert np.max(np.abs(q)) == 127


# ----------------------------------------------------------------- layouts
def test_lmrs_layout(tmp_path):
    s = MF.Shape(dim=64, hidden=96, n_layers=2, n_heads=2, n_kv=1, head_dim=32, ctx=48, eps=1e-6,
                 rope_theta=10000.0)
    p = MF.write_lmrs(str(tmp_path), s, gs=32, seed=9)
    raw = open(p, "rb").read()
    a = L.read_lmrs(p, max_ctx_len=40)
    V = a["shape"][6]
    assert a["shape"] == (64, 96, 2, 2, 1, 32, V, 40) and a["gs"] == 32
    assert a["eps"] == float(np.float32(1e-6)) and a["rope_theta"] == 10000.0
    assert a["end"] == len(raw)
    # the embedding is q * scale of the first tensor after the 256-byte header
    q0 = np.frombuffer(raw, np.int8, 64, 256)
    s0 = np.frombuffer(raw, np.float32, V * 64 // 32, 256 + V * 64)
    assert np.array_equal(a["embedding"][:64], (q0.astype(np.float32) * np.repeat(s0[:2], 32)))
    # kinds in file order: rms_att x L, wq x L, wk x L, wv x L, wo x L, rms_ffn x L, w1 x L, w2 x L, w3 x L
    sizes = {"q": 64 * 64, "k": 32 * 64, "v": 32 * 64, "o": 64 * 64, "f": 96 * 64}
    off = 256 + V * 64 + V * 64 // 32 * 4 + 2 * 64 * 4
    q8_bytes = lambda c: c + c // 32 * 4    # int8 values then f32 scales per group of 32
    off_wk1 = off + 2 * q8_bytes(sizes["q"]) + q8_bytes(sizes["k"])
    assert np.array_equal(a["layers"][1][1][0], np.frombuffer(raw, np.int8, sizes["k"], off_wk1))


def test_safetensors_layout(tmp_path):
    s = MF.Shape(dim=64, hidden=96, n_layers=1, n_heads=2, n_kv=1, head_dim=32, ctx=64)
    p = MF.write_safetensors(str(tmp_path), s, q8_gs=32, seed=4)
    a = L.read_safetensors(p)
    raw = open(p, "rb").read()
    hlen = struct.unpack_from("<Q", raw, 0)[0]
    hdr = json.loads(raw[8:8 + hlen])
    base = 8 + hlen
    e = hdr["model.layers.0.mlp.down_proj.weight"]
    vals = np.frombuffer(raw, np.uint8, 64 * 96, base + e["data_offsets"][0]).reshape(64, 96)
    sc = np.frombuffer(raw, np.float16, 64 * 3, base + hdr["model.layers.0.mlp.down_proj.scales"]["data_offsets"][0])
    bi = np.frombuffer(raw, np.float16, 64 * 3, base + hdr["model.layers.0.mlp.down_proj.biases"]["data_offsets"][0])
    deq = vals.reshape(-1, 32).astype(np.float32) * sc.astype(np.float32)[:, None] + bi.astype(np.float32)[:, None]
    q, sy = a["layers"][0][5]
    assert q.size == 64 * 96 and sy.size == 64 * 3
    assert np.max(np.abs(q.reshape(-1, 32) * sy[:, None] - deq)) <= np.max(sy) / 2 * 1.0001
    assert a["fmt"] == O.Q8_0 and a["gs"] == 32 and a["shape"][7] == 64


# ----------------------------------------------------------------- tokenizers
def test_from_hf_json_pins(tmp_path):
    p = str(tmp_path / "tokenizer.json")
    V = MF.hf_tokenizer_json(p)
    t = OT.OracleTokenizer.from_hf_json(p)
    tokens, merges, hf = bpe_vocab.train()
    n = len(tokens)
    assert len(t.vocab) == V == n + 4
    assert t.vocab[n] == "" and t.vocab[n + 1] == ""           # unused ids stay empty
    assert (t.bos, t.eos) == (n + 2, n + 3) and t.byte_level
    # within one pre-token, score-driven merges equal the HF BPE model's
    table = OT.gpt2_byte_table()
    for word in ["Hello", "world", "quick", "jumps", "assistant", "über", "1234"]:
        mapped = "".join(table[b] for b in word.encode())
        assert t.encode(word) == bpe_vocab.hf_bpe_segment(hf, mapped)
    # no split on the default pre-tokenizer: merges may cross spaces
    assert t.decode(t.encode("Hello, world!  x")) == "Hello, world!  x"


def test_from_hf_json_default_ids(tmp_path):
    p = str(tmp_path / "t.json")
    json.dump({"added_tokens": [{"id": 5, "content": "<x>"}],
               "model": {"vocab": {"a": 0, "b": 1, "ab": 2}, "merges": ["a b"]}}, open(p, "w"))
    t = OT.OracleTokenizer.from_hf_json(p)
    assert t.vocab == ["a", "b", "ab", "", "", "<x>"] and (t.bos, t.eos) == (128000, 128009)


def _write_bin(path, pieces, scores, bos=1, eos=2):
    with open(path, "wb") as f:
        f.write(struct.pack("<4I", len(pieces), 8, bos, eos))
        for p, s in zip(pieces, scores):
            b = p.encode()
            f.write(struct.pack("<fI", s, len(b)) + b)


def test_from_llama2c_hand_cases(tmp_path):
    # ids: 0 <unk> 1 <s> 2 </s>, 3..258 bytes, then t h e a "th" "he" "the"
    pieces = ["<unk>", "<s>", "</s>"] + [f"<0x{b:02X}>" for b in range(256)] + ["t", "h", "e", "a", "th", "he",
                                                                                 "the", " "]
    scores = [0.0] * 259 + [0, 0, 0, 0, -2.0, -1.0, -3.0, 0]
    p = str(tmp_path / "tokenizer.bin")
    _write_bin(p, pieces, scores)
    t = OT.OracleTokenizer.from_llama2c(p)
    T, H, E, A, TH, HE, THE, SP = range(259, 267)
    # "the": "he" (-1) beats "th" (-2); then t + he = "the" is in the vocabulary
    assert t.encode("the") == [THE]
    # "tha": only "th" merges
    assert t.encode("tha", bos=True) == [1, TH, A]
    # "é" is not a piece: its UTF-8 bytes C3 A9 as ids byte + 3
    assert t.encode("té") == [T, 0xC3 + 3, 0xA9 + 3]
    # decode concatenates piece texts (byte pieces stay as their text)
    assert t.decode([THE, SP, 0xC3 + 3, 999]) == "the <0xC3>"
    assert (t.bos, t.eos) == (1, 2)


# library vs oracle ------------------------------------------------------
TEXTS = ["Hello, world!", "the quick brown fox jumps over the lazy dog", "  leading and trailing  ",
         "über café naïve — “quotes”", "中文 文本 😀 🚀", "code: def f(x): return x**2", "a", "\n\n\t ",
         "It's 2024; we'll see 3.14159!", "Hello world, the quick brown fox"]


def test_library_tokenizer_json_matches_oracle(tmp_path):
    import yallma3_mini_inference_amd as Y
    p = str(tmp_path / "tokenizer.json")
    MF.hf_tokenizer_json(p)
    lt, ot = Y.Tokenizer.from_file(p), OT.OracleTokenizer.from_hf_json(p)
    assert lt.vocab_size == len(ot.vocab)
    for s in TEXTS:
        ids = lt.encode(s, bos=True, eos=True)
        assert ids == ot.encode(s, bos=True, eos=True), s
        assert lt.decode(ids[1:-1]) == ot.decode(ids[1:-1]) == s
    r = np.random.default_rng(0)
    for _ in range(20):
        ids = r.integers(0, len(ot.vocab) + 3, 12).tolist()
        assert lt.decode(ids) == ot.decode(ids)
    assert lt.chat_prompt("hi there") == ot.chat_prompt("hi there")


def test_library_tokenizer_bin_matches_oracle(tmp_path):
    import yallma3_mini_inference_amd as Y
    p = str(tmp_path / "tokenizer.bin")
    MF.llama2c_tokenizer_bin(p, n_pad=3)
    lt, ot = Y.Tokenizer.from_file(p), OT.OracleTokenizer.from_llama2c(p)
    assert lt.vocab_size == len(ot.vocab)
    for s in TEXTS:
        ids = lt.encode(s, bos=True)
        assert ids == ot.encode(s, bos=True), s
        assert lt.decode(ids) == ot.decode(ids)
    assert lt.chat_prompt("Hello world") == ot.chat_prompt("Hello world")


# ------------------------------------------------- forward composition
@pytest.mark.parametrize("kind", ["lmrs_gs64", "st_q8_gs32", "st_f16"])
def test_forward_matches_float64(tmp_path, kind):
    """The oracle's forward on lm.rs / safetensors models (HF RoPE with the
    llama3 scaling, the file's group size, F16 chains) against an
    independent float64 forward: within 1e-5 of the logits' scale, while
    plausible mistakes computed the same way differ by more than 1e-4."""
    import formats_np as FN
    s = MF.Shape(dim=64, hidden=128, n_layers=2, n_heads=4, n_kv=2, head_dim=16, ctx=48, rope_theta=10000.0)
    d = str(tmp_path / kind)
    if kind == "lmrs_gs64":
        p = MF.write_lmrs(d, s, gs=64, seed=11)
        arrays, loader = L.read_lmrs(p), L.load_lmrs
    elif kind == "st_q8_gs32":
        p = MF.write_safetensors(d, s, q8_gs=32, seed=12, tokenizer="bin")
        arrays, loader = L.read_safetensors(p), L.load_safetensors
    else:
        p = MF.write_safetensors(d, s, seed=13, tokenizer="bin")
        arrays, loader = L.read_safetensors(p), L.load_safetensors
    m, _ = loader(p)
    sess = m.create_session()
    toks = [3, 17, 250, 5, 99, 42, 7, 300, 11, 64]
    variants = ["reference", "rope_gguf_pairs", "no_llama3_scaling", "gate_up_swapped"]
    if kind == "lmrs_gs64":
        variants.append("group_32")
    refs = {v: FN.Float64Model(arrays, v) for v in variants}
    worst = {v: 0.0 for v in variants}
    for pos, t in enumerate(toks):
        lo = m.forward_x(np.array([t], np.uint32), pos, sess).astype(np.float64)
        scale = np.max(np.abs(lo))
        for v, f in refs.items():
            worst[v] = max(worst[v], float(np.max(np.abs(f.step(t) - lo)) / scale))
    assert worst["reference"] < 1e-5, worst
    for v in variants[1:]:
        assert worst[v] > 1e-4, (v, worst)
