"""ctypes wrapper of the CPU oracle (yl_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg, never by the product package.  Each wrapper
names the reference function it restates (paths relative to the reference
repository).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_BUILD = os.path.join(_HERE, "build")

Q8_0, Q4_0, F16 = 0, 1, 2

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")


def _host_has_avx512() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            txt = f.read()
    except OSError:
        return False
    return all(flag in txt for flag in ("avx512f", "avx512bw", "avx512vl", "avx512dq"))


def build() -> None:
    """Compile the oracle with its Makefile (gcc; no GPU toolchain)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib_path() -> str:
    """The build for this host (v4 with AVX-512, else v3), or the one the
    environment names: YL_ORACLE_ISA = v4 | v3 | sse2 (the thread count is
    OpenMP's OMP_NUM_THREADS)."""
    isa = os.environ.get("YL_ORACLE_ISA") or ("v4" if _host_has_avx512() else "v3")
    if isa not in ("v4", "v3", "sse2"):
        raise ValueError(f"YL_ORACLE_ISA={isa}: expected v4, v3 or sse2")
    return os.path.join(_BUILD, f"liboracle_{isa}.so")


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not os.path.exists(path):
        raise RuntimeError(f"oracle library {path} is not built: run `make -C oracle`")
    L = C.CDLL(path)
    L.yo_f16_to_f32.argtypes = [C.c_uint16]
    L.yo_f16_to_f32.restype = C.c_float
    L.yo_expf.argtypes = [C.c_float]
    L.yo_expf.restype = C.c_float
    L.yo_quantize.argtypes = [C.c_int, _i8p, _f32p, _f32p, _f32p, C.c_size_t, C.c_uint32]
    L.yo_quantize.restype = C.c_int
    L.yo_matmul_q8_slices.argtypes = [_f32p, _i8p, _f32p, _i8p, _f32p, C.c_size_t, C.c_size_t,
                                      C.c_size_t, C.c_size_t]
    L.yo_matmul_f32.argtypes = [_f32p, _f32p, _f32p, C.c_size_t, C.c_size_t, C.c_size_t]
    L.yo_rmsnorm.argtypes = [_f32p, _f32p, _f32p, C.c_size_t, C.c_float]
    L.yo_rope_cos_sin.argtypes = [C.c_void_p, C.c_uint32, _f32p, _f32p]
    L.yo_rope_gguf.argtypes = [C.c_void_p, _f32p, _f32p, C.c_uint32]
    L.yo_fused_attention.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, C.c_size_t, C.c_size_t,
                                     C.c_size_t, C.c_size_t, C.c_size_t, C.c_uint32, C.c_size_t,
                                     C.c_float]
    L.yo_swiglu.argtypes = [_f32p, _f32p, C.c_size_t]
    L.yo_logits.argtypes = [_f32p, _f32p, C.c_void_p, C.c_size_t, C.c_size_t]
    L.yo_argmax.argtypes = [_f32p, C.c_size_t]
    L.yo_argmax.restype = C.c_uint32
    L.yo_model_load.argtypes = [C.c_char_p, C.c_uint32, C.c_int]
    L.yo_model_load.restype = C.c_void_p
    L.yo_model_free.argtypes = [C.c_void_p]
    L.yo_last_error.restype = C.c_char_p
    L.yo_model_shape.argtypes = [C.c_void_p, _u32p]
    L.yo_model_rope_theta.argtypes = [C.c_void_p]
    L.yo_model_rope_theta.restype = C.c_float
    L.yo_model_embedding.argtypes = [C.c_void_p]
    L.yo_model_embedding.restype = C.c_void_p
    L.yo_session_new.argtypes = [C.c_void_p]
    L.yo_session_new.restype = C.c_void_p
    L.yo_session_reset.argtypes = [C.c_void_p]
    L.yo_session_free.argtypes = [C.c_void_p]
    L.yo_session_key_cache.argtypes = [C.c_void_p]
    L.yo_session_key_cache.restype = C.c_void_p
    L.yo_session_value_cache.argtypes = [C.c_void_p]
    L.yo_session_value_cache.restype = C.c_void_p
    L.yo_forward_x.argtypes = [C.c_void_p, _u32p, C.c_size_t, C.c_uint32, C.c_void_p, C.c_void_p]
    L.yo_forward_x.restype = C.c_int
    L.yo_num_threads.restype = C.c_int
    L.yo_rope_hf.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.c_float, C.c_uint32, _f32p, _f32p, C.c_uint32]
    L.yo_model_new.argtypes = [_u32p, C.c_float, C.c_float, C.c_uint32, C.c_int, C.c_int, _f32p, _f32p]
    L.yo_model_new.restype = C.c_void_p
    L.yo_model_set_norms.argtypes = [C.c_void_p, C.c_uint32, _f32p, _f32p]
    L.yo_model_set_weight.argtypes = [C.c_void_p, C.c_uint32, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_size_t]
    _lib = L
    return L


class RopeParams(C.Structure):
    """yo_rope_params: the TransformerShape fields rope_gguf reads (util.rs:653-663)."""
    _fields_ = [("head_size", C.c_uint32), ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32),
                ("rope_theta", C.c_float), ("freq_scale", C.c_float), ("ext_factor", C.c_float),
                ("attn_factor", C.c_float), ("original_ctx_len", C.c_uint32)]


def f16_to_f32(bits: int) -> float:
    return lib().yo_f16_to_f32(bits)


def expf(x: float) -> float:
    return lib().yo_expf(x)


def quantize(fmt: int, x: np.ndarray, gs: int = 32):
    """weight_type::quantize (weight_type.rs:76-90) -> (q int8, scales f32)."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    q = np.zeros(x.size, np.int8)
    s = np.zeros(max(1, x.size // gs), np.float32)
    f = np.zeros(max(1, x.size), np.float32)
    if lib().yo_quantize(fmt, q, s, f, x, x.size, gs) != 0:
        raise ValueError("quantize failed")
    if fmt == F16:
        return f[: x.size], None
    return q, s[: x.size // gs]


def matmul_q8_slices(out, x, x_scale, w, w_scale, n, o, gs=32):
    """weight_type::matmul_q8_slices (weight_type.rs:122-226); out is updated in place."""
    batch = out.size // o
    lib().yo_matmul_q8_slices(out, np.ascontiguousarray(x, np.int8), np.ascontiguousarray(x_scale, np.float32),
                              np.ascontiguousarray(w, np.int8), np.ascontiguousarray(w_scale, np.float32),
                              n, o, gs, batch)
    return out


def matmul_f32(out, x, w, n, o):
    lib().yo_matmul_f32(out, np.ascontiguousarray(x, np.float32), np.ascontiguousarray(w, np.float32),
                        n, o, out.size // o)
    return out


def rmsnorm(x, weight, eps):
    """util::rmsnorm (util.rs:389-426); unwritten tail elements stay 0."""
    x = np.ascontiguousarray(x, np.float32)
    o = np.zeros_like(x)
    lib().yo_rmsnorm(o, x, np.ascontiguousarray(weight, np.float32), x.size, eps)
    return o


def rope_params(head_size, n_heads, n_kv_heads, theta, freq_scale=1.0, ext_factor=0.0,
                attn_factor=1.0, original_ctx_len=4096) -> RopeParams:
    return RopeParams(head_size, n_heads, n_kv_heads, theta, freq_scale, ext_factor, attn_factor,
                      original_ctx_len)


def rope_cos_sin(p: RopeParams, pos: int):
    c = np.zeros(p.head_size // 2, np.float32)
    s = np.zeros(p.head_size // 2, np.float32)
    lib().yo_rope_cos_sin(C.byref(p), pos, c, s)
    return c, s


def rope_gguf(p: RopeParams, q, k, pos):
    """util::rope_gguf (util.rs:653-718), in place on q and k."""
    lib().yo_rope_gguf(C.byref(p), q, k, pos)


def fused_attention(sq, key_cache, value_cache, seq_len, batch, n_heads, n_kv_heads, head_size,
                    start_pos, kv_dim, attn_scale):
    """forward.rs fused_attention (forward.rs:299-400) -> output [batch*n_heads*head_size]."""
    out = np.zeros(batch * n_heads * head_size, np.float32)
    scores = np.zeros(n_heads * batch * seq_len, np.float32)
    lib().yo_fused_attention(out, scores, np.ascontiguousarray(sq, np.float32),
                             np.ascontiguousarray(key_cache, np.float32),
                             np.ascontiguousarray(value_cache, np.float32), seq_len, batch, n_heads,
                             n_kv_heads, head_size, start_pos, kv_dim, attn_scale)
    return out


def swiglu(gate, up):
    g = np.array(gate, np.float32, copy=True)
    lib().yo_swiglu(g, np.ascontiguousarray(up, np.float32), g.size)
    return g


def logits(last, emb, vocab, dim):
    out = np.zeros(vocab, np.float32)
    emb = np.ascontiguousarray(emb, np.float32)
    lib().yo_logits(out, np.ascontiguousarray(last, np.float32), emb.ctypes.data, vocab, dim)
    return out


def argmax(p) -> int:
    return int(lib().yo_argmax(np.ascontiguousarray(p, np.float32), len(p)))


def rope_hf(sq, k, head_size, n_heads, n_kv_heads, rope_theta, ctx_len, pos):
    """util::rope (util.rs:589-635) on one token's q and k, in place."""
    lib().yo_rope_hf(head_size, n_heads, n_kv_heads, rope_theta, ctx_len, sq, k, pos)


def num_threads() -> int:
    return int(lib().yo_num_threads())


class Model:
    """TransformerLlamaGguf restated (transformer_llama_gguf.rs:183-729)."""

    def __init__(self, path: str | None = None, max_ctx_len: int = 0xFFFFFFFF, fmt_override: int = -1, handle=None):
        self._h = handle if handle is not None else lib().yo_model_load(path.encode(), max_ctx_len, fmt_override)
        if not self._h:
            raise RuntimeError("oracle load failed: " + lib().yo_last_error().decode())
        shp = np.zeros(8, np.uint32)
        lib().yo_model_shape(self._h, shp)
        (self.dim, self.hidden, self.n_layers, self.n_heads, self.n_kv_heads, self.head_size,
         self.vocab, self.ctx_len) = (int(v) for v in shp)
        self.kv_dim = self.n_kv_heads * self.head_size

    @classmethod
    def from_arrays(cls, shape, eps, rope_theta, gs, hf_rope, fmt, embedding, rms_final, rms_att, rms_ffn, layers):
        """A model from loader output (oracle/loaders.py): shape = (dim, hidden,
        n_layers, n_heads, n_kv_heads, head_size, vocab, ctx_len); layers[l] =
        7 projections (q, k, v, o, gate, down, up), each (q int8, s f32) for
        Q8_0 or an f32 array for F16."""
        h = lib().yo_model_new(np.array(shape, np.uint32), eps, rope_theta, gs, int(hf_rope), fmt,
                               np.ascontiguousarray(embedding, np.float32), np.ascontiguousarray(rms_final, np.float32))
        for l, projs in enumerate(layers):
            lib().yo_model_set_norms(h, l, np.ascontiguousarray(rms_att[l], np.float32),
                                     np.ascontiguousarray(rms_ffn[l], np.float32))
            for k, w in enumerate(projs):
                if fmt == F16:
                    f = np.ascontiguousarray(w, np.float32)
                    lib().yo_model_set_weight(h, l, k, F16, None, None, f.ctypes.data, f.size)
                else:
                    q = np.ascontiguousarray(w[0], np.int8)
                    sc = np.ascontiguousarray(w[1], np.float32)
                    lib().yo_model_set_weight(h, l, k, fmt, q.ctypes.data, sc.ctypes.data, None, q.size)
        return cls(handle=h)

    def close(self):
        if self._h:
            lib().yo_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def embedding(self) -> np.ndarray:
        ptr = lib().yo_model_embedding(self._h)
        buf = (C.c_float * (self.vocab * self.dim)).from_address(ptr)
        return np.frombuffer(buf, np.float32)

    def create_session(self) -> "Session":
        return Session(self)

    def forward_x(self, tokens, start_pos: int, session: "Session") -> np.ndarray:
        """Transformer::forward_x (transformer.rs:53, forward.rs:120-297): last-token logits."""
        toks = np.ascontiguousarray(tokens, np.uint32)
        out = np.zeros(self.vocab, np.float32)
        rc = lib().yo_forward_x(self._h, toks, toks.size, start_pos, session._h, out.ctypes.data)
        if rc != 0:
            raise RuntimeError("oracle forward failed: " + lib().yo_last_error().decode())
        return out


class Session:
    """InferenceSession (base_transformer.rs:81-105)."""

    def __init__(self, model: Model):
        self.model = model
        self._h = lib().yo_session_new(model._h)
        if not self._h:
            raise RuntimeError("oracle session failed: " + lib().yo_last_error().decode())
        self.pos = 0

    def _cache(self, which):
        m = self.model
        n = m.n_layers * m.ctx_len * m.kv_dim
        fn = lib().yo_session_key_cache if which == "k" else lib().yo_session_value_cache
        buf = (C.c_float * n).from_address(fn(self._h))
        return np.frombuffer(buf, np.float32).reshape(m.n_layers, m.ctx_len, m.kv_dim)

    def key_cache(self) -> np.ndarray:
        return self._cache("k")

    def value_cache(self) -> np.ndarray:
        return self._cache("v")

    def reset(self):
        lib().yo_session_reset(self._h)
        self.pos = 0

    def __del__(self):
        try:
            if self._h:
                lib().yo_session_free(self._h)
                self._h = None
        except Exception:
            pass
