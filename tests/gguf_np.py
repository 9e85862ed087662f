"""A GGUF v3 reader and writer in numpy, written for the tests, and an
independent float64 forward pass over the tensors it reads.

This is test infrastructure and shares no code with the oracle or the
library: it parses the file's bytes itself, decodes the blocks the way the
reference's loader does (transformer_llama_gguf.rs:345-410: Q8_0 = f16 d +
32 int8; Q4_0 = f16 d + 16 bytes, byte j's low nibble is element 2j and its
high nibble element 2j+1, unsigned 0..15, no offset), and restates
llama_forward_x (forward.rs:120-280) in float64 with the reference's
activation quantization (quantization.rs:29-52, weight_type.rs:52-74).  It
checks the composition of the oracle's forward pass -- which tensors feed
which step, in which order -- to a tolerance, not its f32 bits.
"""
from __future__ import annotations

import struct

import numpy as np

GGUF_MAGIC = 0x46554747
T_F32, T_F16, T_Q4_0, T_Q8_0 = 0, 1, 2, 8

# metadata value types
_U8, _I8, _U16, _I16, _U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _I64, _F64 = range(13)
_SCALAR = {_U8: "<B", _I8: "<b", _U16: "<H", _I16: "<h", _U32: "<I", _I32: "<i", _F32: "<f", _BOOL: "<B",
           _U64: "<Q", _I64: "<q", _F64: "<d"}


class Reader:
    def __init__(self, data: bytes):
        self.d, self.o = data, 0

    def take(self, fmt):
        v = struct.unpack_from(fmt, self.d, self.o)[0]
        self.o += struct.calcsize(fmt)
        return v

    def string(self):
        n = self.take("<Q")
        s = self.d[self.o:self.o + n].decode("utf-8", errors="replace")
        self.o += n
        return s

    def value(self, t):
        if t == _STR:
            return self.string()
        if t == _ARR:
            et, n = self.take("<I"), self.take("<Q")
            return [self.value(et) for _ in range(n)]
        return self.take(_SCALAR[t])


class Gguf:
    """Metadata and tensor views of one GGUF v3 file."""

    def __init__(self, path: str):
        with open(path, "rb") as f:
            self.data = f.read()
        r = Reader(self.data)
        assert r.take("<I") == GGUF_MAGIC, "bad magic"
        assert r.take("<I") == 3, "GGUF version 3 only"
        n_t, n_kv = r.take("<Q"), r.take("<Q")
        self.meta, self.meta_type = {}, {}
        for _ in range(n_kv):
            k = r.string()
            t = r.take("<I")
            self.meta[k] = r.value(t)
            self.meta_type[k] = t
        infos = []
        for _ in range(n_t):
            name = r.string()
            nd = r.take("<I")
            dims = [r.take("<Q") for _ in range(nd)]
            typ, off = r.take("<I"), r.take("<Q")
            infos.append((name, dims, typ, off))
        align = int(self.meta.get("general.alignment", 32))
        start = (r.o + align - 1) // align * align
        self.tensors = {n: (dims, typ, start + off) for n, dims, typ, off in infos}

    def n_elements(self, name):
        return int(np.prod(self.tensors[name][0]))

    def raw(self, name):
        dims, typ, off = self.tensors[name]
        n = self.n_elements(name)
        size = {T_F32: 4 * n, T_F16: 2 * n, T_Q8_0: n // 32 * 34, T_Q4_0: n // 32 * 18}[typ]
        return np.frombuffer(self.data, np.uint8, size, off), typ

    def quantized(self, name, q4_order="reference"):
        """(values, block scales as float64): Q8_0 int8 values, Q4_0 nibbles 0..15.
        q4_order "ggml" decodes Q4_0 the way GGML does (element j in the low
        nibble of byte j, j + 16 in its high nibble, minus 8) -- a plausible
        misreading the tests use as a negative control."""
        raw, typ = self.raw(name)
        if typ == T_Q8_0:
            b = raw.reshape(-1, 34)
            d = b[:, :2].copy().view(np.float16).astype(np.float64).ravel()
            return b[:, 2:].copy().view(np.int8).astype(np.int64).ravel(), d
        if typ == T_Q4_0:
            b = raw.reshape(-1, 18)
            d = b[:, :2].copy().view(np.float16).astype(np.float64).ravel()
            by = b[:, 2:].astype(np.int64)
            q = np.empty((b.shape[0], 32), np.int64)
            if q4_order == "ggml":
                q[:, :16] = (by & 0x0F) - 8
                q[:, 16:] = (by >> 4) - 8
                return q.ravel(), d
            q[:, 0::2] = by & 0x0F      # element 2j: low nibble of byte j
            q[:, 1::2] = by >> 4        # element 2j + 1: high nibble
            return q.ravel(), d
        raise ValueError(f"{name}: type {typ} is not a block format")

    def f32(self, name):
        raw, typ = self.raw(name)
        if typ == T_F32:
            return raw.copy().view(np.float32).astype(np.float64)
        if typ == T_F16:
            return raw.copy().view(np.float16).astype(np.float64)
        v, d = self.quantized(name)
        return v.astype(np.float64) * np.repeat(d, 32)

    def tensor_type(self, name):
        return self.tensors[name][1]


# ------------------------------------------------------------------ writer

def _pack_value(t, v):
    if t == _STR:
        b = v.encode()
        return struct.pack("<Q", len(b)) + b
    if t == _ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_pack_value(et, x) for x in items)
    return struct.pack(_SCALAR[t], v)


def q8_blocks(qs: np.ndarray, d_f16: np.ndarray) -> bytes:
    """Q8_0 blocks from int8 values [n] and f16 scales [n/32]."""
    qs = np.asarray(qs, np.int8).reshape(-1, 32)
    out = np.zeros((qs.shape[0], 34), np.uint8)
    out[:, :2] = np.asarray(d_f16, np.float16).reshape(-1, 1).view(np.uint8)
    out[:, 2:] = qs.view(np.uint8)
    return out.tobytes()


def q4_blocks(nibbles: np.ndarray, d_f16: np.ndarray) -> bytes:
    """Q4_0 blocks from unsigned values 0..15 [n] in element order (element
    2j into the low nibble of byte j, 2j + 1 into its high nibble)."""
    v = np.asarray(nibbles, np.uint8).reshape(-1, 32)
    assert v.max(initial=0) < 16
    out = np.zeros((v.shape[0], 18), np.uint8)
    out[:, :2] = np.asarray(d_f16, np.float16).reshape(-1, 1).view(np.uint8)
    out[:, 2:] = v[:, 0::2] | (v[:, 1::2] << 4)
    return out.tobytes()


def write(path: str, meta: list, tensors: list, alignment: int = 32) -> None:
    """meta: [(key, type, value)] (arrays as (elem_type, items)); tensors:
    [(name, dims, ggml_type, bytes)] with dims in GGUF order (row length
    first)."""
    head = struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(meta))
    kv = b"".join(_pack_value(_STR, k) + struct.pack("<I", t) + _pack_value(t, v) for k, t, v in meta)
    infos, off, blobs = b"", 0, []
    for name, dims, typ, blob in tensors:
        infos += _pack_value(_STR, name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", typ, off)
        pad = (-len(blob)) % alignment
        blobs.append(blob + b"\0" * pad)
        off += len(blob) + pad
    pre = head + kv + infos
    pre += b"\0" * ((-len(pre)) % alignment)
    with open(path, "wb") as f:
        f.write(pre)
        for b in blobs:
            f.write(b)


def llama_meta(dim, hidden, n_layers, n_heads, n_kv_heads, vocab, ctx, file_type=7, rope_theta=10000.0,
               eps=1e-5, rope_scaling=None, attention_scale=None):
    """rope_scaling: (factor, ext_factor, attn_factor, original_context_length)
    written as the llama.rope.scaling.* keys; attention_scale as
    llama.attention.scale."""
    meta = [("general.architecture", _STR, "llama"), ("general.file_type", _U32, file_type),
            ("llama.embedding_length", _U32, dim), ("llama.feed_forward_length", _U32, hidden),
            ("llama.block_count", _U32, n_layers), ("llama.attention.head_count", _U32, n_heads),
            ("llama.attention.head_count_kv", _U32, n_kv_heads), ("llama.context_length", _U32, ctx),
            ("llama.rope.freq_base", _F32, rope_theta), ("llama.attention.layer_norm_rms_epsilon", _F32, eps),
            ("tokenizer.ggml.tokens", _ARR, (_STR, [f"<t{i}>" for i in range(vocab)]))]
    if rope_scaling is not None:
        f, e, a, n = rope_scaling
        meta += [("llama.rope.scaling.factor", _F32, f), ("llama.rope.scaling.ext_factor", _F32, e),
                 ("llama.rope.scaling.attn_factor", _F32, a),
                 ("llama.rope.scaling.original_context_length", _U32, n)]
    if attention_scale is not None:
        meta.append(("llama.attention.scale", _F32, attention_scale))
    return meta


# ------------------------------------------------- float64 forward (forward.rs)

def _quantize(x, fmt):
    """Q8_0 (quantization.rs:29-52): d = absmax/127, q = round(x/d) half away
    from zero; Q4_0 (weight_type.rs:52-74): d = absmax/7, clamp to +-7.
    Returns the dequantized values q*d per 32-group, as the matmul sees them
    once the integer dot is scaled (the block sum of q_x*q_w is exact)."""
    g = np.asarray(x, np.float64).reshape(-1, 32)
    qmax = 127.0 if fmt == T_Q8_0 else 7.0
    d = np.abs(g).max(axis=1) / qmax
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(d[:, None] > 0, g / d[:, None], 0.0)
    q = np.sign(r) * np.floor(np.abs(r) + 0.5)
    q = np.clip(q, -7, 7) if fmt == T_Q4_0 else np.clip(q, -128, 127)
    return q, d


def _matmul(x, w_q, w_d, fmt, rows, cols):
    """out[c] = sum_b (sum_k qx*qw) * dw * dx for one activation row."""
    qx, dx = _quantize(x, fmt)
    W = w_q.reshape(rows, cols // 32, 32).astype(np.float64)
    isum = np.einsum("bk,rbk->rb", qx, W)
    return (isum * w_d.reshape(rows, cols // 32) * dx[None, :]).sum(axis=1)


def _rmsnorm(x, w, eps):
    return w * (x / np.sqrt(np.mean(x * x) + eps))


def _rope_pairs(v, c, s, head_size, neox=False):
    """rope_gguf's rotation (util.rs:653-718) with pair k's (cos, sin):
    consecutive pairs (2k, 2k+1) of every head.  neox=True pairs
    (k, k + head_size/2) instead (the HF layout, a negative control)."""
    if neox:
        out = v.copy().reshape(-1, 2, head_size // 2)
        a, b = out[:, 0].copy(), out[:, 1].copy()
        out[:, 0] = a * c - b * s
        out[:, 1] = a * s + b * c
        return out.reshape(-1)
    out = v.copy().reshape(-1, head_size // 2, 2)
    a, b = out[..., 0].copy(), out[..., 1].copy()
    out[..., 0] = a * c - b * s
    out[..., 1] = a * s + b * c
    return out.reshape(-1)


YARN_VARIANTS = ("yarn_interp_in_mix", "yarn_no_floor", "yarn_no_attn_factor", "yarn_ramp_reversed")


def yarn_cos_sin(pos, head_size, base, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0, n_ctx_orig=4096,
                 variant="reference"):
    """rope_gguf's per-pair (cos, sin) (util.rs:653-724) in float64, from the
    closed form of the angle: pair k's base angle is pos * base^(-2k/head_size)
    (the reference's `theta *= theta_scale` recurrence, unrounded).  With
    freq_scale = 1/factor, YaRN's ramp between the correction dims
    low = max(floor(head_size * ln(n_ctx_orig / (2 pi * 32)) / (2 ln base)), 0)
    and high = min(low, c) + min(c, head_size/2) - low, where
    c = head_size * ln(n_ctx_orig / (2 pi)) / (2 ln base), gives
    ramp(k) = 1 - clamp((k - low) / max(high - low, 0.001), 0, 1) and the angle
    t = freq_scale*theta*(1 - ramp*ext) + theta*ramp*ext; both are scaled by
    attn_factor.  A `variant` from YARN_VARIANTS plants one mistake: the mix
    with freq_scale*theta in place of theta, corr_start without floor, no
    attn_factor, or the ramp reversed."""
    n_pairs = head_size // 2
    k = np.arange(n_pairs, dtype=np.float64)
    theta = pos * float(base) ** (-2.0 * k / head_size)
    ln_b2 = 2.0 * np.log(float(base))
    cs = head_size * np.log(n_ctx_orig / (2.0 * np.pi * 32.0)) / ln_b2
    low = max(cs if variant == "yarn_no_floor" else np.floor(cs), 0.0)
    ce = head_size * np.log(n_ctx_orig / (2.0 * np.pi)) / ln_b2
    high = min(low, ce) + min(ce, float(n_pairs)) - max(low, 0.0)
    interp = freq_scale * theta
    t = interp
    if ext_factor != 0.0:
        ramp = 1.0 - np.clip((k - low) / max(high - low, 0.001), 0.0, 1.0)
        if variant == "yarn_ramp_reversed":
            ramp = 1.0 - ramp
        mix = ramp * ext_factor
        t = interp * (1.0 - mix) + (interp if variant == "yarn_interp_in_mix" else theta) * mix
    a = 1.0 if variant == "yarn_no_attn_factor" else attn_factor
    return a * np.cos(t), a * np.sin(t)


# mistakes visible on any model, and those that need the YaRN keys and
# llama.attention.scale to be present
BASE_VARIANTS = ("q4_ggml_order", "rope_neox", "gate_up_swapped", "norms_swapped", "no_attn_scale")
SCALING_VARIANTS = YARN_VARIANTS + ("attention_scale_ignored",)
VARIANTS = ("reference",) + BASE_VARIANTS + SCALING_VARIANTS


class Float64Model:
    """llama_forward_x in float64 over a Gguf (single-format or per-tensor).
    `variant` other than "reference" computes one plausible mistake, for the
    tests that show the oracle does not agree with it."""

    def __init__(self, g: Gguf, variant: str = "reference"):
        assert variant in VARIANTS
        m = g.meta
        self.g = g
        self.variant = variant
        self.dim = int(m["llama.embedding_length"])
        self.hidden = int(m["llama.feed_forward_length"])
        self.n_layers = int(m["llama.block_count"])
        self.n_heads = int(m["llama.attention.head_count"])
        self.n_kv = int(m.get("llama.attention.head_count_kv", self.n_heads))
        self.hd = self.dim // self.n_heads
        self.kv_dim = self.n_kv * self.hd
        self.eps = float(m["llama.attention.layer_norm_rms_epsilon"])
        self.theta = float(m.get("llama.rope.freq_base", 10000.0))
        # YaRN keys and the attention scale (transformer_llama_gguf.rs:242-249)
        raw = float(m.get("llama.rope.scaling.factor", 1.0))
        self.freq_scale = 1.0 / raw if raw != 0.0 else 1.0
        self.ext_factor = float(m.get("llama.rope.scaling.ext_factor", 0.0))
        self.attn_factor = float(m.get("llama.rope.scaling.attn_factor", 1.0))
        self.n_ctx_orig = int(m.get("llama.rope.scaling.original_context_length", m["llama.context_length"]))
        self.attention_scale = float(m.get("llama.attention.scale", 0.0))
        self.vocab = len(m["tokenizer.ggml.tokens"])
        order = "ggml" if variant == "q4_ggml_order" else "reference"
        if g.tensor_type("token_embd.weight") in (T_Q8_0, T_Q4_0):
            q, d = g.quantized("token_embd.weight", order)
            self.emb = (q.astype(np.float64) * np.repeat(d, 32)).reshape(self.vocab, self.dim)
        else:
            self.emb = g.f32("token_embd.weight").reshape(self.vocab, self.dim)
        self.w = {}
        for l in range(self.n_layers):
            for nm in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"):
                t = f"blk.{l}.{nm}.weight"
                q, d = g.quantized(t, order)
                self.w[(l, nm)] = (q, d, g.tensor_type(t))
            na, nf = "attn_norm", "ffn_norm"
            if variant == "norms_swapped":
                na, nf = nf, na
            self.w[(l, "attn_norm")] = g.f32(f"blk.{l}.{na}.weight")
            self.w[(l, "ffn_norm")] = g.f32(f"blk.{l}.{nf}.weight")
        self.out_norm = g.f32("output_norm.weight")
        self.k = np.zeros((self.n_layers, 0, self.kv_dim))
        self.v = np.zeros((self.n_layers, 0, self.kv_dim))

    def _mm(self, l, name, x, rows, cols):
        q, d, fmt = self.w[(l, name)]
        return _matmul(x, q, d, fmt, rows, cols)

    def step(self, token: int) -> np.ndarray:
        """One token at the next position; returns float64 logits."""
        pos = self.k.shape[1]
        x = self.emb[token].copy() if token < self.vocab else np.zeros(self.dim)
        att = self.n_heads * self.hd
        newk = np.zeros((self.n_layers, 1, self.kv_dim))
        newv = np.zeros((self.n_layers, 1, self.kv_dim))
        for l in range(self.n_layers):
            xn = _rmsnorm(x, self.w[(l, "attn_norm")], self.eps)
            q = self._mm(l, "attn_q", xn, att, self.dim)
            k = self._mm(l, "attn_k", xn, self.kv_dim, self.dim)
            v = self._mm(l, "attn_v", xn, self.kv_dim, self.dim)
            neox = self.variant == "rope_neox"
            c, sn = yarn_cos_sin(pos, self.hd, self.theta, self.freq_scale, self.ext_factor, self.attn_factor,
                                 self.n_ctx_orig, self.variant)
            q, k = _rope_pairs(q, c, sn, self.hd, neox), _rope_pairs(k, c, sn, self.hd, neox)
            newk[l, 0], newv[l, 0] = k, v
            K = np.concatenate([self.k[l], k[None]], 0)
            V = np.concatenate([self.v[l], v[None]], 0)
            out = np.zeros(att)
            r = self.n_heads // self.n_kv
            for h in range(self.n_heads):
                kvh = h // r
                sl = slice(kvh * self.hd, (kvh + 1) * self.hd)
                s = K[:, sl] @ q[h * self.hd:(h + 1) * self.hd]
                if self.attention_scale != 0.0 and self.variant != "attention_scale_ignored":
                    s = s * self.attention_scale   # llama.attention.scale (forward.rs:142-146)
                elif self.variant != "no_attn_scale":
                    s = s / np.sqrt(self.hd)
                p = np.exp(s - s.max())
                p /= p.sum()
                out[h * self.hd:(h + 1) * self.hd] = p @ V[:, sl]
            x = x + self._mm(l, "attn_output", out, self.dim, att)
            xn = _rmsnorm(x, self.w[(l, "ffn_norm")], self.eps)
            gate = self._mm(l, "ffn_gate", xn, self.hidden, self.dim)
            up = self._mm(l, "ffn_up", xn, self.hidden, self.dim)
            if self.variant == "gate_up_swapped":
                gate, up = up, gate
            h_ = gate / (1.0 + np.exp(-gate)) * up
            x = x + self._mm(l, "ffn_down", h_, self.dim, self.hidden)
        self.k = np.concatenate([self.k, newk], 1)
        self.v = np.concatenate([self.v, newv], 1)
        return self.emb @ _rmsnorm(x, self.out_norm, self.eps)


# ------------------------------------------ small random models (test inputs)

def _rand_q8(rng, rows, cols, std):
    w = rng.normal(0, std, (rows * cols // 32, 32))
    d = (np.abs(w).max(axis=1) / 127.0).astype(np.float16)
    df = d.astype(np.float64)
    q = np.where(df[:, None] > 0, np.round(w / np.where(df > 0, df, 1)[:, None]), 0)
    return q8_blocks(np.clip(q, -127, 127).astype(np.int8), d)


def _rand_q4(rng, rows, cols, std):
    n = rows * cols // 32
    # GGML writes d = (signed absmax) / -8, so block scales take either sign
    d = (rng.uniform(std / 8, std / 4, n) * rng.choice([-1.0, 1.0], n)).astype(np.float16)
    return q4_blocks(rng.integers(0, 16, (n, 32)), d)


def random_llama(path, dim=64, hidden=128, n_layers=2, n_heads=2, n_kv_heads=1, vocab=96, ctx=64,
                 attn_fmt=T_Q8_0, ffn_fmt=T_Q8_0, embd_fmt=T_Q8_0, seed=0, rope_theta=10000.0,
                 nan_embedding_rows=(), nan_output_norm=False, emb_std=0.5, w_std=0.05, rope_scaling=None,
                 attention_scale=None):
    """A random llama GGUF whose norm weights differ per tensor (so a swapped
    norm changes the result), with optional NaN block scales in chosen rows
    of the token embedding or a NaN final-norm weight."""
    rng = np.random.default_rng(seed)
    att, kv = dim, dim // n_heads * n_kv_heads

    def qt(name, rows, cols, fmt, std=w_std):
        blob = _rand_q8(rng, rows, cols, std) if fmt == T_Q8_0 else _rand_q4(rng, rows, cols, std)
        return (name, [cols, rows], fmt, blob)

    def norm(name, n):
        return (name, [n], T_F32, rng.uniform(0.5, 1.5, n).astype(np.float32).tobytes())

    emb = qt("token_embd.weight", vocab, dim, embd_fmt, emb_std)
    if nan_embedding_rows:
        bs = 34 if embd_fmt == T_Q8_0 else 18
        raw = bytearray(emb[3])
        for r in nan_embedding_rows:
            for b in range(dim // 32):
                o = (r * (dim // 32) + b) * bs
                raw[o:o + 2] = np.array([np.nan], np.float16).tobytes()
        emb = emb[:3] + (bytes(raw),)
    tensors = [emb]
    on = norm("output_norm.weight", dim)
    if nan_output_norm:
        on = on[:3] + (np.full(dim, np.nan, np.float32).tobytes(),)
    tensors.append(on)
    for l in range(n_layers):
        p = f"blk.{l}."
        tensors += [norm(p + "attn_norm.weight", dim), norm(p + "ffn_norm.weight", dim),
                    qt(p + "attn_q.weight", att, dim, attn_fmt), qt(p + "attn_k.weight", kv, dim, attn_fmt),
                    qt(p + "attn_v.weight", kv, dim, attn_fmt), qt(p + "attn_output.weight", dim, att, attn_fmt),
                    qt(p + "ffn_gate.weight", hidden, dim, ffn_fmt), qt(p + "ffn_down.weight", dim, hidden, ffn_fmt),
                    qt(p + "ffn_up.weight", hidden, dim, ffn_fmt)]
    ft = 2 if attn_fmt == ffn_fmt == T_Q4_0 else 7
    write(path, llama_meta(dim, hidden, n_layers, n_heads, n_kv_heads, vocab, ctx, file_type=ft,
                           rope_theta=rope_theta, rope_scaling=rope_scaling, attention_scale=attention_scale),
          tensors)
    return path


def swap_tensors(src, dst, a, b):
    """Copy of a GGUF with the data of tensors a and b exchanged (same type and size)."""
    g = Gguf(src)
    ra, ta = g.raw(a)
    rb, tb = g.raw(b)
    assert ta == tb and ra.size == rb.size
    data = bytearray(g.data)
    oa, ob = g.tensors[a][2], g.tensors[b][2]
    data[oa:oa + ra.size], data[ob:ob + rb.size] = bytes(rb), bytes(ra)
    with open(dst, "wb") as f:
        f.write(bytes(data))
    return dst
