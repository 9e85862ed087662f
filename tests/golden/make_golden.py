"""Writes tests/golden/forward_golden.npz: the oracle's end-to-end results on
seeded random llama GGUFs built by tests/gguf_np.py (Q8_0, Q4_0, Q8_0
attention beside a Q4_0 FFN, and Q8_0 with YaRN RoPE scaling and an explicit
attention scale).  Per model: a prompt's last-token logits, 12
greedy token ids after it, and the logits of the last greedy step.

    python tests/golden/make_golden.py      (rewrites the fixture)

tests/test_oracle_pins.py recomputes the same values with the oracle and
requires them bit for bit; tests/test_gpu_pins.py requires them of the HIP
path.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import gguf_np as G  # noqa: E402

FIXTURE = os.path.join(HERE, "forward_golden.npz")
STEPS = 12
MODELS = {
    # name: (attention, FFN, embedding formats, seed, prompt length)
    "q8": (G.T_Q8_0, G.T_Q8_0, G.T_Q8_0, 21, 9),
    "q4": (G.T_Q4_0, G.T_Q4_0, G.T_Q4_0, 22, 17),
    "mixed": (G.T_Q8_0, G.T_Q4_0, G.T_Q8_0, 23, 70),
    "yarn": (G.T_Q8_0, G.T_Q8_0, G.T_Q8_0, 24, 40),
}
# GGUF keys beyond the shape: YaRN RoPE scaling (factor 4 from an original
# context of 2048, ext_factor 1, attn_factor 1.2) and llama.attention.scale
EXTRA = {"yarn": dict(rope_scaling=(4.0, 1.0, 1.2, 2048), attention_scale=0.15)}


def model_path(name, directory):
    a, f, e, seed, _ = MODELS[name]
    return G.random_llama(os.path.join(directory, f"golden_{name}.gguf"), dim=128, hidden=256, n_layers=2,
                          n_heads=4, n_kv_heads=2, vocab=300, ctx=128, attn_fmt=a, ffn_fmt=f, embd_fmt=e,
                          seed=seed, rope_theta=500000.0, emb_std=0.05, w_std=0.2, **EXTRA.get(name, {}))


def prompt(name):
    _, _, _, seed, n = MODELS[name]
    return np.random.default_rng(seed).integers(0, 300, n).astype(np.uint32)


def compute(oracle, directory):
    out = {}
    for name in MODELS:
        m = oracle.Model(model_path(name, directory))
        s = m.create_session()
        p = prompt(name)
        lo = m.forward_x(p, 0, s)
        out[f"{name}_prompt"] = p
        out[f"{name}_prefill_logits"] = lo
        tok, ids = oracle.argmax(lo), []
        for i in range(STEPS):
            lo = m.forward_x([tok], len(p) + i, s)
            tok = oracle.argmax(lo)
            ids.append(tok)
        out[f"{name}_greedy"] = np.array(ids, np.uint32)
        out[f"{name}_last_logits"] = lo
    return out


if __name__ == "__main__":
    import tempfile
    from oracle import oracle as O
    if not os.path.exists(O.lib_path()):
        O.build()
    with tempfile.TemporaryDirectory() as d:
        res = compute(O, d)
    np.savez(FIXTURE, **res)
    print(f"wrote {FIXTURE}: " + ", ".join(f"{k}{tuple(v.shape)}" for k, v in res.items()))
