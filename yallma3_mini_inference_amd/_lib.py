"""ctypes binding of libyallma3_amd.so (declarations: include/yallma3.h).

The shared library is the product: HIP kernels for gfx950 plus the C++ host
runtime.  There is no fallback -- if the library is not built this module
raises, and every compute call goes through the HIP path.
"""
from __future__ import annotations

import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "lib", "libyallma3_amd.so")

YL_OK = 0
STATUS_NAMES = {
    -1: "YL_ERR_ARG", -2: "YL_ERR_FORMAT", -3: "YL_ERR_IO", -4: "YL_ERR_GGUF", -5: "YL_ERR_HIP",
    -6: "YL_ERR_UNSUPPORTED", -7: "YL_ERR_NOMEM", -8: "YL_ERR_RANGE",
}

# every symbol include/yallma3.h declares
EXPORTS = [
    "yl_last_error", "load_transformer_ffi", "infer_ffi", "free_string", "yl_ffi_model", "yl_device_count", "yl_malloc",
    "yl_free", "yl_memcpy_h2d", "yl_memcpy_d2h", "yl_memcpy_d2d", "yl_matmul_bench", "yl_memset_d", "yl_synchronize", "yl_quantize",
    "yl_weight_upload", "yl_weight_upload_gguf", "yl_weight_free", "yl_weight_bytes", "yl_matmul",
    "yl_rmsnorm_quantize", "yl_rope_gguf", "yl_attention", "yl_attention_split", "yl_attention_noalloc", "yl_swiglu_quantize", "yl_load",
    "yl_model_free", "yl_model_name", "yl_model_shape", "yl_vocab_size", "yl_max_ctx_len", "yl_bos_token",
    "yl_eos_token", "yl_model_weight_bytes", "yl_model_embedding_bytes", "yl_get_embeddings",
    "yl_create_session", "yl_session_free", "yl_session_reset", "yl_session_set_attention", "yl_session_pos", "yl_session_set_pos",
    "yl_session_kv", "yl_forward_x", "yl_generate_greedy", "yl_profile_kernel", "yl_profile_step", "yl_profile_stream", "yl_math_selftest", "yl_serial_sum_selftest", "yl_wait_fault_selftest",
    "yl_write_synthetic_gguf", "yl_synthetic_normal", "yl_write_synthetic_gguf_tok", "yl_infer_set_max_tokens",
    "yl_infer_reset", "yl_tokenizer_load", "yl_tokenizer_free", "yl_model_tokenizer", "yl_tokenizer_vocab_size",
    "yl_tokenize", "yl_detokenize", "yl_chat_template", "yl_chat_prompt", "yl_pretokenize", "yl_sampler_new",
    "yl_sampler_sample", "yl_sampler_free", "yl_generate_text", "yl_weight_upload_f16", "yl_matmul_f32",
]


class YlError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class RopeParams(C.Structure):
    _fields_ = [("head_size", C.c_uint32), ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32),
                ("rope_theta", C.c_float), ("freq_scale", C.c_float), ("ext_factor", C.c_float),
                ("attn_factor", C.c_float), ("original_ctx_len", C.c_uint32)]


class Shape(C.Structure):
    """yl_shape: TransformerShape (base_transformer.rs:25-44)."""
    _fields_ = [("dimension", C.c_uint32), ("hidden_dimension", C.c_uint32), ("n_heads", C.c_uint32),
                ("head_size", C.c_uint32), ("n_kv_heads", C.c_uint32), ("vocab_size", C.c_uint32),
                ("n_layers", C.c_uint32), ("ctx_len", C.c_uint32), ("rms_norm_eps", C.c_float),
                ("rope_theta", C.c_float), ("group_size", C.c_uint32), ("rope_freq_scale", C.c_float),
                ("rope_ext_factor", C.c_float), ("rope_attn_factor", C.c_float),
                ("rope_original_ctx_len", C.c_uint32), ("attention_scale", C.c_float),
                ("weight_format", C.c_int32)]


class SynthConfig(C.Structure):
    _fields_ = [("dim", C.c_uint32), ("hidden", C.c_uint32), ("n_layers", C.c_uint32), ("n_heads", C.c_uint32),
                ("n_kv_heads", C.c_uint32), ("vocab", C.c_uint32), ("ctx_len", C.c_uint32),
                ("rope_theta", C.c_float), ("rms_eps", C.c_float), ("weight_std", C.c_float),
                ("attn_format", C.c_int32), ("ffn_format", C.c_int32), ("embd_format", C.c_int32),
                ("file_type", C.c_int32), ("seed", C.c_uint64), ("rope_scaling", C.c_int32),
                ("rope_scaling_factor", C.c_float), ("rope_ext_factor", C.c_float), ("rope_attn_factor", C.c_float),
                ("rope_original_ctx", C.c_uint32), ("attention_scale", C.c_float)]


class SynthTokenizer(C.Structure):
    _fields_ = [("tokens", C.POINTER(C.c_char_p)), ("n_tokens", C.c_size_t), ("merges", C.POINTER(C.c_char_p)),
                ("n_merges", C.c_size_t), ("bos", C.c_uint32), ("eos", C.c_uint32), ("pre", C.c_char_p),
                ("chat_template", C.c_char_p), ("add_bos_token", C.c_int32), ("add_space_prefix", C.c_int32)]


_lib = None


def lib():
    """Load the library (raises if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built: run `python -m yallma3_mini_inference_amd.build`")
    L = C.CDLL(LIB_PATH)
    vp, sz, st = C.c_void_p, C.c_size_t, C.c_int32
    u32, u64, f32 = C.c_uint32, C.c_uint64, C.c_float
    sig = {
        "yl_last_error": (C.c_char_p, []),
        "load_transformer_ffi": (C.c_bool, [C.c_char_p]),
        "infer_ffi": (vp, [C.c_char_p]),
        "free_string": (None, [vp]),
        "yl_ffi_model": (vp, []),
        "yl_device_count": (st, [C.POINTER(C.c_int)]),
        "yl_malloc": (vp, [sz]),
        "yl_free": (None, [vp]),
        "yl_memcpy_h2d": (st, [vp, vp, sz]),
        "yl_memcpy_d2h": (st, [vp, vp, sz]),
        "yl_memcpy_d2d": (st, [vp, vp, sz]),
        "yl_matmul_bench": (st, [vp, sz, vp, vp, sz, vp, u32, C.POINTER(C.c_double)]),
        "yl_memset_d": (st, [vp, C.c_int, sz]),
        "yl_synchronize": (st, []),
        "yl_quantize": (st, [C.c_int, vp, vp, vp, sz, u32, vp]),
        "yl_weight_upload": (vp, [C.c_int, vp, vp, sz, sz]),
        "yl_weight_upload_gguf": (vp, [C.c_int, vp, sz, sz]),
        "yl_weight_free": (None, [vp]),
        "yl_weight_bytes": (sz, [vp]),
        "yl_matmul": (st, [vp, C.c_int, vp, vp, sz, vp, sz, sz, u32, vp]),
        "yl_rmsnorm_quantize": (st, [vp, vp, sz, f32, sz, vp, st, vp, vp, vp]),
        "yl_rope_gguf": (st, [C.POINTER(RopeParams), vp, vp, sz, u32, vp]),
        "yl_attention": (st, [vp, vp, vp, vp, sz, u32, u32, u32, u32, f32, vp]),
        "yl_attention_split": (st, [vp, vp, vp, vp, u32, u32, u32, u32, f32, vp]),
        "yl_attention_noalloc": (st, [vp, vp, vp, vp, sz, u32, u32, u32, u32, f32, vp]),
        "yl_swiglu_quantize": (st, [vp, vp, sz, sz, vp, st, vp, vp, vp]),
        "yl_load": (vp, [C.c_char_p, u32, st]),
        "yl_model_free": (None, [vp]),
        "yl_model_name": (C.c_char_p, [vp]),
        "yl_model_shape": (st, [vp, C.POINTER(Shape)]),
        "yl_vocab_size": (sz, [vp]),
        "yl_max_ctx_len": (u32, [vp]),
        "yl_bos_token": (u32, [vp]),
        "yl_eos_token": (u32, [vp]),
        "yl_model_weight_bytes": (sz, [vp]),
        "yl_model_embedding_bytes": (sz, [vp]),
        "yl_get_embeddings": (st, [vp, vp, sz, vp]),
        "yl_create_session": (vp, [vp]),
        "yl_session_free": (None, [vp]),
        "yl_session_reset": (st, [vp]),
        "yl_session_set_attention": (st, [vp, C.c_int32]),
        "yl_session_pos": (u32, [vp]),
        "yl_session_set_pos": (None, [vp, u32]),
        "yl_session_kv": (st, [vp, C.POINTER(vp), C.POINTER(vp), C.POINTER(sz)]),
        "yl_forward_x": (st, [vp, vp, sz, u32, vp, vp, vp]),
        "yl_generate_greedy": (st, [vp, vp, u32, u32, u32, vp]),
        "yl_profile_step": (st, [vp, vp, u32, u32, st, u32, C.POINTER(C.c_double)]),
        "yl_profile_stream": (st, [vp, vp, st, u32, C.POINTER(C.c_double), C.POINTER(u64)]),
        "yl_profile_kernel": (st, [vp, vp, u32, u32, u32, st, u32, C.POINTER(C.c_double), C.POINTER(u64),
                                   C.POINTER(u32)]),
        "yl_math_selftest": (st, [vp, sz, vp, vp, vp, vp]),
        "yl_serial_sum_selftest": (st, [vp, vp, sz, u32, vp]),
        "yl_wait_fault_selftest": (st, []),
        "yl_write_synthetic_gguf": (st, [C.c_char_p, C.POINTER(SynthConfig)]),
        "yl_synthetic_normal": (st, [u64, u64, u64, sz, f32, vp]),
        "yl_write_synthetic_gguf_tok": (st, [C.c_char_p, C.POINTER(SynthConfig), C.POINTER(SynthTokenizer)]),
        "yl_infer_set_max_tokens": (None, [u32]),
        "yl_infer_reset": (None, []),
        "yl_tokenizer_load": (vp, [C.c_char_p]),
        "yl_tokenizer_free": (None, [vp]),
        "yl_model_tokenizer": (vp, [vp]),
        "yl_tokenizer_vocab_size": (sz, [vp]),
        "yl_tokenize": (st, [vp, C.c_char_p, st, st, vp, sz, C.POINTER(sz)]),
        "yl_detokenize": (st, [vp, vp, sz, vp, sz, C.POINTER(sz)]),
        "yl_chat_template": (st, [vp, st, C.c_char_p, st, vp, sz, C.POINTER(sz)]),
        "yl_chat_prompt": (st, [vp, C.c_char_p, vp, sz, C.POINTER(sz)]),
        "yl_pretokenize": (st, [C.c_char_p, vp, sz, C.POINTER(sz)]),
        "yl_sampler_new": (vp, [sz, f32, f32, u64]),
        "yl_sampler_sample": (st, [vp, vp, C.POINTER(u32)]),
        "yl_sampler_free": (None, [vp]),
        "yl_generate_text": (st, [vp, vp, vp, vp, sz, u32, C.POINTER(vp), vp, sz, C.POINTER(sz)]),
        "yl_weight_upload_f16": (vp, [vp, sz, sz]),
        "yl_matmul_f32": (st, [vp, vp, sz, vp, sz, sz, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def last_error() -> str:
    return (lib().yl_last_error() or b"").decode(errors="replace")


def check(status: int) -> None:
    if status != YL_OK:
        raise YlError(status, last_error())
