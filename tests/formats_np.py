"""A float64 forward pass for lm.rs and safetensors models (test
infrastructure), written from the mathematics and the reference's formulas,
not from the oracle: quantization in groups of gs (quantization.rs:29-52)
for Q8 files, none for F16 (matmul_f32, weight_type.rs:228-270), HF-layout
RoPE with the llama3 frequency scaling (util.rs:589-635), softmax attention,
SwiGLU and tied logits (forward.rs:120-280).  `variant` other than
"reference" computes one plausible mistake, for the tests that show the
oracle does not agree with it.
"""
from __future__ import annotations

import math

import numpy as np

VARIANTS = ("reference", "rope_gguf_pairs", "no_llama3_scaling", "gate_up_swapped", "group_32")


def _quant_groups(x, gs):
    """q * d per group of gs (the matmul's exact integer dots, rescaled)."""
    g = np.asarray(x, np.float64).reshape(-1, gs)
    d = np.abs(g).max(axis=1) / 127.0
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(d[:, None] > 0, g / d[:, None], 0.0)
    q = np.clip(np.sign(r) * np.floor(np.abs(r) + 0.5), -128, 127)
    return (q * d[:, None]).reshape(-1)


def _freqs(head, theta, ctx, scaled=True):
    out = []
    for j in range(head // 2):
        f = theta ** (-(2.0 * j) / head)
        if scaled:
            wl = 2 * math.pi / f
            if wl > ctx:
                f = f / 32.0
            elif wl >= ctx / 4.0:
                s = (ctx / wl - 1.0) / 3.0
                f = (1 - s) * f / 32.0 + s * f
        out.append(f)
    return np.array(out)


def _rope(v, pos, head, freqs, hf=True):
    ang = pos * freqs
    c, s = np.cos(ang), np.sin(ang)
    if hf:
        o = v.copy().reshape(-1, 2, head // 2)
        a, b = o[:, 0].copy(), o[:, 1].copy()
        o[:, 0], o[:, 1] = a * c - b * s, a * s + b * c
    else:
        o = v.copy().reshape(-1, head // 2, 2)
        a, b = o[..., 0].copy(), o[..., 1].copy()
        o[..., 0], o[..., 1] = a * c - b * s, a * s + b * c
    return o.reshape(-1)


class Float64Model:
    """arrays = the dict of oracle.loaders.read_lmrs / read_safetensors."""

    def __init__(self, arrays: dict, variant: str = "reference"):
        assert variant in VARIANTS
        self.v = variant
        (self.dim, self.hidden, self.nl, self.nh, self.nkv, self.hd, self.vocab, self.ctx) = arrays["shape"]
        self.eps, self.q8 = arrays["eps"], arrays["fmt"] != 2
        self.gs = 32 if variant == "group_32" else arrays["gs"]
        self.emb = np.asarray(arrays["embedding"], np.float64).reshape(self.vocab, self.dim)
        self.rms_att = [np.asarray(w, np.float64) for w in arrays["rms_att"]]
        self.rms_ffn = [np.asarray(w, np.float64) for w in arrays["rms_ffn"]]
        self.rms_final = np.asarray(arrays["rms_final"], np.float64)
        gsw = arrays["gs"]
        self.W = []
        for projs in arrays["layers"]:
            mats = []
            for w in projs:
                if self.q8:
                    q, s = w
                    mats.append(q.astype(np.float64) * np.repeat(np.asarray(s, np.float64), gsw))
                else:
                    mats.append(np.asarray(w, np.float64))
            self.W.append(mats)
        self.freqs = _freqs(self.hd, arrays["rope_theta"], self.ctx, variant != "no_llama3_scaling")
        self.K = [np.zeros((0, self.nkv * self.hd)) for _ in range(self.nl)]
        self.V = [np.zeros((0, self.nkv * self.hd)) for _ in range(self.nl)]

    def _mm(self, w, x, rows):
        xq = _quant_groups(x, self.gs) if self.q8 else x
        return w.reshape(rows, -1) @ xq

    def step(self, token: int) -> np.ndarray:
        pos = self.K[0].shape[0]
        att, kvd, hd = self.nh * self.hd, self.nkv * self.hd, self.hd
        x = self.emb[token].copy()
        hf = self.v != "rope_gguf_pairs"
        for l in range(self.nl):
            wq, wk, wv, wo, w1, w2, w3 = self.W[l]
            xn = self.rms_att[l] * (x / np.sqrt(np.mean(x * x) + self.eps))
            q = _rope(self._mm(wq, xn, att), pos, hd, self.freqs, hf)
            k = _rope(self._mm(wk, xn, kvd), pos, hd, self.freqs, hf)
            v = self._mm(wv, xn, kvd)
            self.K[l] = np.concatenate([self.K[l], k[None]])
            self.V[l] = np.concatenate([self.V[l], v[None]])
            out = np.zeros(att)
            r = self.nh // self.nkv
            for h in range(self.nh):
                sl = slice((h // r) * hd, (h // r + 1) * hd)
                s = self.K[l][:, sl] @ q[h * hd:(h + 1) * hd] / math.sqrt(hd)
                p = np.exp(s - s.max())
                out[h * hd:(h + 1) * hd] = (p / p.sum()) @ self.V[l][:, sl]
            x = x + self._mm(wo, out, self.dim)
            xn = self.rms_ffn[l] * (x / np.sqrt(np.mean(x * x) + self.eps))
            g, u = self._mm(w1, xn, self.hidden), self._mm(w3, xn, self.hidden)
            if self.v == "gate_up_swapped":
                g, u = u, g
            x = x + self._mm(w2, g / (1.0 + np.exp(-g)) * u, self.dim)
        xn = self.rms_final * (x / np.sqrt(np.mean(x * x) + self.eps))
        return self.emb @ xn
