"""MI355X-native quantized LLaMA forward path (yaLLMa3 mini-inference).

Compute runs in libyallma3_amd.so (HIP kernels for gfx950 + C++ host,
C ABI in include/yallma3.h); this package is the Python mirror of the
reference's API over it:

  WeightFormat, QuantizedWeight, quantize, matmul      weight_type.rs
  Transformer (TransformerLlamaGguf), InferenceSession transformer.rs,
                                                       base_transformer.rs
  load_transformer, load_transformer_ffi, infer_ffi    lib.rs, README.md
  Tokenizer, Sampler                                   tokenizer.rs, sampler.rs
  ops.*                                                util.rs, forward.rs
  synth                                                seeded GGUF models
"""
from ._lib import LIB_PATH, YlError, check, lib
from .device import DeviceBuffer, device_count
from .tokenizer import Sampler, Tokenizer, pretokenize
from .transformer import (InferenceSession, Transformer, TransformerLlamaGguf, infer_ffi, infer_reset,
                          infer_set_max_tokens, load_transformer, load_transformer_ffi)
from .weight_type import QuantizedWeight, WeightFormat, matmul, matmul_device, quantize, quantize_device

__all__ = [
    "LIB_PATH", "YlError", "check", "lib", "DeviceBuffer", "device_count", "InferenceSession", "Transformer",
    "TransformerLlamaGguf", "infer_ffi", "load_transformer", "load_transformer_ffi", "QuantizedWeight",
    "WeightFormat", "matmul", "matmul_device", "quantize", "quantize_device", "Sampler", "Tokenizer", "pretokenize",
    "infer_reset", "infer_set_max_tokens",
]
