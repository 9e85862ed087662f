"""The Transformer trait and InferenceSession over the HIP forward path.

Python mirror of the reference's model API:
  load_transformer(path, ...)     lib.rs:107-133 (.gguf, .lmrs, .safetensors)
  Transformer                     trait Transformer, transformer.rs:19-69,
                                  implemented as TransformerLlamaGguf
                                  (transformer_llama_gguf.rs:658-729)
  InferenceSession                base_transformer.rs:81-105 (KV cache on
                                  the device; `pos` kept for the caller)
  load_transformer_ffi / infer_ffi
                                  lib.rs:135-152, README.md:81-92
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from ._lib import Shape, YlError, check, last_error, lib
from .tokenizer import Sampler, Tokenizer
from .weight_type import WeightFormat


class InferenceSession:
    """Per-conversation state: device KV cache [n_layers][ctx_len][kv_dim] and `pos`."""

    def __init__(self, model: "Transformer"):
        self.model = model
        self._h = lib().yl_create_session(model._h)
        if not self._h:
            raise YlError(-5, last_error())

    @property
    def pos(self) -> int:
        return int(lib().yl_session_pos(self._h))

    @pos.setter
    def pos(self, value: int) -> None:
        lib().yl_session_set_pos(self._h, int(value))

    def reset(self) -> None:
        """InferenceSession::reset (base_transformer.rs:100-104)."""
        check(lib().yl_session_reset(self._h))

    def set_attention(self, mode: str) -> None:
        """Decode attention of this session: "exact" (fused_attention,
        forward.rs:299-400, in the reference's operation order) or "split"
        (the same quantity with the context split over many workgroups;
        differs in rounding only, for a tolerance bar)."""
        modes = {"exact": 0, "split": 1}
        if mode not in modes:
            raise ValueError(f"attention mode must be one of {sorted(modes)}")
        check(lib().yl_session_set_attention(self._h, modes[mode]))

    def _kv(self):
        k, v, n = C.c_void_p(), C.c_void_p(), C.c_size_t()
        check(lib().yl_session_kv(self._h, C.byref(k), C.byref(v), C.byref(n)))
        return k.value, v.value, n.value

    def key_cache(self) -> np.ndarray:
        """Keys [n_layers][ctx_len][kv_dim] (the device holds them transposed)."""
        ctx = self.model.shape.ctx_len
        k = self._download(self._kv()[0], transposed=True)
        return np.ascontiguousarray(k[:, :, :ctx].transpose(0, 2, 1))

    def value_cache(self) -> np.ndarray:
        """Values [n_layers][ctx_len][kv_dim]."""
        return np.ascontiguousarray(self._download(self._kv()[1])[:, :self.model.shape.ctx_len])

    def _shape(self, transposed=False):
        """Device cache shape; kv_ld = ctx_len rounded up to a multiple of 4."""
        m = self.model
        ld, kv = (m.shape.ctx_len + 3) & ~3, m.shape.n_kv_heads * m.shape.head_size
        return (m.shape.n_layers, kv, ld) if transposed else (m.shape.n_layers, ld, kv)

    def _download(self, ptr, transposed=False) -> np.ndarray:
        out = np.empty(self._shape(transposed), np.float32)
        check(lib().yl_memcpy_d2h(out.ctypes.data, ptr, out.nbytes))
        return out

    def upload_kv(self, key: np.ndarray, value: np.ndarray) -> None:
        """Overwrite the device KV cache from [n_layers][P][kv_dim] arrays of
        the first P <= ctx_len positions (the rest become zeros); tests and
        benchmarks pre-fill it."""
        kp, vp, n = self._kv()
        m = self.model
        kv = m.shape.n_kv_heads * m.shape.head_size
        key = np.asarray(key, np.float32)
        value = np.asarray(value, np.float32)
        P = key.size // (m.shape.n_layers * kv)
        if key.size != m.shape.n_layers * P * kv or value.size != key.size or P > m.shape.ctx_len:
            raise ValueError("cache shape mismatch")
        shp = (m.shape.n_layers, P, kv)
        kd = np.zeros(self._shape(True), np.float32)
        kd[:, :, :P] = key.reshape(shp).transpose(0, 2, 1)
        vd = np.zeros(self._shape(), np.float32)
        vd[:, :P] = value.reshape(shp)
        for ptr, a in ((kp, kd), (vp, vd)):
            if a.size != n:
                raise ValueError("cache shape mismatch")
            check(lib().yl_memcpy_h2d(ptr, a.ctypes.data, a.nbytes))

    def close(self) -> None:
        if self._h:
            lib().yl_session_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Transformer:
    """TransformerLlamaGguf / TransformerLlamaLmrs / TransformerLlamaSt on one
    MI355X (the file's extension picks the loader; name() says which)."""

    def __init__(self, path: str, max_ctx_len: int = 0xFFFFFFFF, fmt_override: WeightFormat | None = None):
        ov = -1 if fmt_override is None else int(fmt_override)
        self._h = lib().yl_load(os.fsencode(path), max_ctx_len, ov)
        if not self._h:
            raise YlError(-4, last_error())
        self.shape = Shape()
        check(lib().yl_model_shape(self._h, C.byref(self.shape)))

    # trait Transformer, transformer.rs:19-69
    @classmethod
    def load_model(cls, model_path: str, max_ctx_len: int) -> "Transformer":
        return cls(model_path, max_ctx_len)

    def name(self) -> str:
        return lib().yl_model_name(self._h).decode()

    def vocab_size(self) -> int:
        return int(lib().yl_vocab_size(self._h))

    def get_embeddings(self, token: int) -> np.ndarray:
        return self.get_embeddings_batch([token])[0]

    def get_embeddings_batch(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.uint32)
        out = np.zeros((t.size, self.shape.dimension), np.float32)
        check(lib().yl_get_embeddings(self._h, t.ctypes.data, t.size, out.ctypes.data))
        return out

    def forward_x(self, tokens, start_pos: int, session: InferenceSession) -> np.ndarray:
        """Logits (vocab f32) of the last token; K/V accumulate into the session cache."""
        t = np.ascontiguousarray(tokens, np.uint32)
        logits = np.empty(self.vocab_size(), np.float32)
        check(lib().yl_forward_x(self._h, t.ctypes.data, t.size, int(start_pos), session._h, logits.ctypes.data,
                                 None))
        return logits

    def forward_argmax(self, tokens, start_pos: int, session: InferenceSession) -> int:
        """forward_x followed by greedy sampling on the device (no logits copy)."""
        t = np.ascontiguousarray(tokens, np.uint32)
        out = C.c_uint32(0)
        check(lib().yl_forward_x(self._h, t.ctypes.data, t.size, int(start_pos), session._h, None, C.byref(out)))
        return int(out.value)

    def generate_greedy(self, session: InferenceSession, token: int, start_pos: int, n_steps: int) -> np.ndarray:
        """n_steps single-token forward_x calls chained on the device by argmax."""
        out = np.zeros(n_steps, np.uint32)
        check(lib().yl_generate_greedy(self._h, session._h, int(token), int(start_pos), int(n_steps),
                                       out.ctypes.data))
        return out

    # kernel classes of yl_profile_kernel
    PROFILE_CLASSES = {"qkv": 0, "attention": 1, "wo": 2, "w13": 3, "w2": 4, "logits": 5}

    def profile_kernel(self, session: InferenceSession, token: int, start_pos: int, kernel_class: str,
                       reps: int = 20, batch: int = 1):
        """Average launch time (us), bytes per launch and launches per step of one
        kernel class, from a graph of that class's launches of one step over
        `batch` tokens replayed `reps` times between two HIP events.  Modifies
        the session's state at those positions (reset it afterwards)."""
        us, nbytes, n = C.c_double(), C.c_uint64(), C.c_uint32()
        check(lib().yl_profile_kernel(self._h, session._h, int(token), int(start_pos), int(batch),
                                      self.PROFILE_CLASSES[kernel_class], int(reps), C.byref(us),
                                      C.byref(nbytes), C.byref(n)))
        return us.value, nbytes.value, n.value

    def profile_step(self, session: InferenceSession, token: int, start_pos: int, skip_class: str | None = None,
                     reps: int = 20):
        """Time (us) of one decode step at start_pos as its graph launches it,
        without the launches of skip_class (None: the whole step), from
        `reps` replays between two HIP events.  Modifies the session's state
        at that position (reset it afterwards)."""
        us = C.c_double()
        cls = -1 if skip_class is None else self.PROFILE_CLASSES[skip_class]
        check(lib().yl_profile_step(self._h, session._h, int(token), int(start_pos), cls, int(reps), C.byref(us)))
        return us.value

    def profile_stream(self, session: InferenceSession, kernel_class: str, reps: int = 20):
        """Plain stream of one GEMV class's weights with that GEMV's grid, per
        layer, replayed as a graph: (us per launch, bytes per launch)."""
        us, nbytes = C.c_double(), C.c_uint64()
        check(lib().yl_profile_stream(self._h, session._h, self.PROFILE_CLASSES[kernel_class], int(reps),
                                      C.byref(us), C.byref(nbytes)))
        return us.value, nbytes.value

    def create_session(self) -> InferenceSession:
        return InferenceSession(self)

    def tokenizer(self) -> Tokenizer:
        """Transformer::tokenizer (transformer.rs): the GGUF's tokenizer."""
        return Tokenizer(lib().yl_model_tokenizer(self._h), owner=self)

    def generate_text(self, session: InferenceSession, sampler: Sampler, prompt_ids, max_tokens: int = 0):
        """One chat turn's generation (main.rs:186-216) from session.pos:
        returns (text, generated ids); session.pos advances."""
        t = np.ascontiguousarray(prompt_ids, np.uint32)
        cap = max_tokens if max_tokens else self.max_ctx_len()
        ids = np.zeros(max(cap, 1), np.uint32)
        text, n = C.c_void_p(), C.c_size_t()
        check(lib().yl_generate_text(self._h, session._h, sampler._h, t.ctypes.data, t.size, int(max_tokens),
                                     C.byref(text), ids.ctypes.data, ids.size, C.byref(n)))
        try:
            out = C.string_at(text.value).decode()
        finally:
            lib().free_string(text)
        return out, [int(x) for x in ids[:min(n.value, ids.size)]]

    def max_ctx_len(self) -> int:
        return int(lib().yl_max_ctx_len(self._h))

    def eos_token(self) -> int:
        return int(lib().yl_eos_token(self._h))

    def bos_token(self) -> int:
        return int(lib().yl_bos_token(self._h))

    def weight_bytes(self) -> int:
        return int(lib().yl_model_weight_bytes(self._h))

    def embedding_bytes(self) -> int:
        return int(lib().yl_model_embedding_bytes(self._h))

    def close(self) -> None:
        if self._h:
            lib().yl_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


TransformerLlamaGguf = Transformer


def load_transformer(model_path: str, sequential: bool = False, max_ctx_len: int = 0xFFFFFFFF,
                     fmt_override: WeightFormat | None = None) -> Transformer:
    """lib.rs:107-133: ".gguf" (TransformerLlamaGguf), ".lmrs"
    (TransformerLlamaLmrs) and ".safetensors" (TransformerLlamaSt) files.
    sequential=True with a safetensors file asks for the reference's scalar
    teaching forward (TransformerLlamaStSeq), which is not built here."""
    ext = os.path.splitext(model_path)[1].lstrip(".")
    if ext not in ("gguf", "lmrs", "safetensors"):
        raise YlError(-6, f"Unsupported model extension for path: {model_path}")
    if ext == "safetensors" and sequential:
        raise YlError(-6, "TransformerLlamaStSeq (the sequential scalar forward) is not built; "
                          "load with sequential=False")
    return Transformer(model_path, max_ctx_len, fmt_override)


def load_transformer_ffi(model_path: str | None) -> bool:
    return bool(lib().load_transformer_ffi(None if model_path is None else os.fsencode(model_path)))


def infer_set_max_tokens(n: int) -> None:
    lib().yl_infer_set_max_tokens(int(n))


def infer_reset() -> None:
    lib().yl_infer_reset()


def infer_ffi(prompt: str) -> str | None:
    p = lib().infer_ffi(prompt.encode())
    if not p:
        return None
    try:
        return C.string_at(p).decode(errors="replace")
    finally:
        lib().free_string(p)
