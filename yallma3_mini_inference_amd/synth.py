"""Seeded synthetic GGUF llama models of the benchmark shapes.

    python -m yallma3_mini_inference_amd.synth llama32_1b /tmp/l1.gguf

Weights ~N(0, 0.02), RMSNorm weights 1.0, placeholder vocabulary strings;
written by the library's host-side generator (yl_write_synthetic_gguf), so
the same (config, seed) gives the same bytes on every machine.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import os
import sys

from ._lib import SynthConfig, SynthTokenizer, check, lib
from .weight_type import WeightFormat

Q8, Q4, F16 = WeightFormat.Q8_0, WeightFormat.Q4_0, WeightFormat.F16


@dataclasses.dataclass(frozen=True)
class ModelConfig:
    dim: int
    hidden: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    vocab: int
    ctx_len: int
    rope_theta: float = 10000.0
    rms_eps: float = 1e-5
    weight_std: float = 0.02
    attn_format: int = Q8
    ffn_format: int = Q8
    embd_format: int = Q8
    file_type: int = 7
    seed: int = 0
    # llama.rope.scaling.{factor, ext_factor, attn_factor, original_context_length}
    # (written when not None) and llama.attention.scale (written when nonzero)
    rope_scaling: tuple | None = None
    attention_scale: float = 0.0

    def to_c(self) -> SynthConfig:
        sc = self.rope_scaling or (0.0, 0.0, 0.0, 0)
        return SynthConfig(self.dim, self.hidden, self.n_layers, self.n_heads, self.n_kv_heads, self.vocab,
                           self.ctx_len, self.rope_theta, self.rms_eps, self.weight_std, int(self.attn_format),
                           int(self.ffn_format), int(self.embd_format), self.file_type, self.seed,
                           1 if self.rope_scaling else 0, sc[0], sc[1], sc[2], int(sc[3]), self.attention_scale)


CONFIGS = {
    # small shapes the CPU oracle finishes in seconds
    "tiny": ModelConfig(128, 256, 2, 4, 2, 512, 256),
    "tiny_q4": ModelConfig(128, 256, 2, 4, 2, 512, 256, attn_format=Q4, ffn_format=Q4, file_type=2),
    "tiny_mixed": ModelConfig(128, 384, 3, 4, 1, 1000, 300, rope_theta=500000.0, ffn_format=Q4),
    # dim 96: the embedding table's rows are padded to 128 (zero-scale blocks); vocab 300 ends in a partial tile
    "tiny_pad": ModelConfig(96, 192, 2, 3, 1, 300, 128, seed=3),
    # ctx 4096, the longest context of the single decode attention kernel (head size 64, 4 query heads
    # per kv head): its softmax sum runs on one lane up to 2560 positions and one wavefront beyond
    "tiny_long": ModelConfig(256, 512, 2, 4, 1, 512, 4096, seed=7),
    # head size 64, 2 query heads per kv head, context_length 131072 (a Llama-3.x
    # GGUF's): decode past 16384 positions streams the softmax row in segments
    "tiny_ctx131k": ModelConfig(256, 512, 2, 4, 2, 512, 131072, rope_theta=500000.0, seed=11),
    # head size 32 beside a 20000-position context: its decode attention keeps
    # the scores row in LDS and stops at 16384 positions
    "tiny_hd32_long": ModelConfig(128, 256, 2, 4, 2, 512, 20000, seed=12),
    # ctx 8448 with 4 query heads per kv head (head size 64): decode beyond
    # 4096 positions runs the four-kernel split attention inside the graph
    "tiny_8k": ModelConfig(256, 512, 2, 4, 1, 512, 8448, seed=9),
    # head size 128 with 8 query heads per kv head, and with 1: the split
    # decode attention's widest and narrowest groups
    "tiny_hd128_r8": ModelConfig(1024, 512, 2, 8, 1, 512, 2048, seed=13),
    "tiny_hd128_r1": ModelConfig(256, 512, 2, 2, 2, 512, 2048, seed=14),
    # F16 weights and embedding (general.file_type 1), and a Q8_0 model whose
    # token embedding is F16
    "tiny_f16": ModelConfig(128, 256, 2, 4, 2, 512, 256, attn_format=F16, ffn_format=F16, embd_format=F16,
                            file_type=1, seed=21),
    "tiny_q8_f16emb": ModelConfig(128, 256, 2, 4, 2, 512, 256, embd_format=F16, seed=22),
    "small_f16": ModelConfig(576, 1536, 3, 9, 3, 2048, 1024, attn_format=F16, ffn_format=F16, embd_format=F16,
                             file_type=1, seed=23),
    # SmolLM2-135M shape: dim 576, FFN 1536, 30 layers, 9/3 heads, vocab 49152
    "smollm2_135m": ModelConfig(576, 1536, 30, 9, 3, 49152, 2048),
    # Llama-3.2-1B shape: dim 2048, FFN 8192, 16 layers, 32/8 heads, vocab 128256
    "llama32_1b": ModelConfig(2048, 8192, 16, 32, 8, 128256, 4096, rope_theta=500000.0),
    "llama32_1b_q4": ModelConfig(2048, 8192, 16, 32, 8, 128256, 4096, rope_theta=500000.0, attn_format=Q4,
                                 ffn_format=Q4, file_type=2),
    # YaRN RoPE scaling (factor 4 from an original context of 1024, ext_factor 1,
    # attn_factor 1.1: pairs 0-5 keep the unscaled angle, pairs past 17.7 take
    # the interpolated one, the ramp mixes those between) and an explicit
    # attention scale of 0.11 instead of 1/sqrt(64)
    "tiny_yarn": ModelConfig(256, 512, 2, 4, 2, 512, 4096, seed=31, rope_scaling=(4.0, 1.0, 1.1, 1024),
                             attention_scale=0.11),
    # the same scaling with ext_factor 0.5 (a half-weight ramp) on a Q4_0 model
    "tiny_yarn_q4": ModelConfig(256, 512, 2, 4, 2, 512, 4096, rope_theta=500000.0, attn_format=Q4, ffn_format=Q4,
                                file_type=2, seed=32, rope_scaling=(8.0, 0.5, 0.9, 2048), attention_scale=0.2),
    # Llama-3-8B shape, Q4_0 FFN beside Q8_0 attention, context for 8192 + 256 tokens
    "llama3_8b_mixed": ModelConfig(4096, 14336, 32, 32, 8, 128256, 8448, rope_theta=500000.0, ffn_format=Q4),
    # two layers of that shape (same vocabulary): a prompt chunk's kernels at
    # the 8B layer shape, within the oracle's test time
    "llama3_8b_mixed_2l": ModelConfig(4096, 14336, 2, 32, 8, 128256, 8448, rope_theta=500000.0, ffn_format=Q4,
                                      seed=41),
}


@dataclasses.dataclass(frozen=True)
class TokenizerSpec:
    """GGUF tokenizer metadata for a synthetic model (len(tokens) = vocab)."""
    tokens: tuple
    merges: tuple = ()
    bos: int = 1
    eos: int = 2
    pre: str | None = None
    chat_template: str | None = None
    add_bos_token: bool | None = None
    add_space_prefix: bool | None = None


def write(path: str, cfg: ModelConfig, tokenizer: TokenizerSpec | None = None) -> str:
    c = cfg.to_c()
    if tokenizer is None:
        check(lib().yl_write_synthetic_gguf(os.fsencode(path), C.byref(c)))
        return path
    toks = (C.c_char_p * len(tokenizer.tokens))(*[t.encode() for t in tokenizer.tokens])
    merges = (C.c_char_p * max(1, len(tokenizer.merges)))(*[m.encode() for m in tokenizer.merges])
    tri = lambda v: -1 if v is None else int(v)
    spec = SynthTokenizer(toks, len(tokenizer.tokens), merges, len(tokenizer.merges), tokenizer.bos, tokenizer.eos,
                          None if tokenizer.pre is None else tokenizer.pre.encode(),
                          None if tokenizer.chat_template is None else tokenizer.chat_template.encode(),
                          tri(tokenizer.add_bos_token), tri(tokenizer.add_space_prefix))
    check(lib().yl_write_synthetic_gguf_tok(os.fsencode(path), C.byref(c), C.byref(spec)))
    return path


def model_dir() -> str:
    d = os.environ.get("YL_MODEL_DIR", os.path.join(os.environ.get("TMPDIR", "/tmp"), "yallma3_models"))
    os.makedirs(d, exist_ok=True)
    return d


def ensure(name: str, directory: str | None = None) -> str:
    """Path of the named synthetic model, written on first use."""
    cfg = CONFIGS[name]
    path = os.path.join(directory or model_dir(), f"{name}_seed{cfg.seed}.gguf")
    if not os.path.exists(path):
        tmp = path + f".tmp{os.getpid()}"
        write(tmp, cfg)
        os.replace(tmp, path)
    return path


if __name__ == "__main__":
    if len(sys.argv) != 3 or sys.argv[1] not in CONFIGS:
        print(f"usage: python -m yallma3_mini_inference_amd.synth <{'|'.join(CONFIGS)}> <out.gguf>")
        sys.exit(2)
    write(sys.argv[2], CONFIGS[sys.argv[1]])
