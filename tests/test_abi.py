"""CPU checks of the product library: it loads, exports every symbol the
header declares, and its host-only pieces (synthetic GGUF writer, normal
generator) behave; the GGUF it writes is readable by the oracle's restated
reference loader.  No GPU compute is called here."""
import hashlib
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def _declared_functions():
    src = open(os.path.join(ROOT, "include", "yallma3.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"\b([a-z_][a-z0-9_]*)\s*\(", src)
    skip = {"if", "sizeof", "defined"}
    return sorted({n for n in names if n not in skip and not n.startswith("__")})


def test_header_symbols_exported(yl):
    import ctypes
    from yallma3_mini_inference_amd import _lib
    lib = ctypes.CDLL(_lib.LIB_PATH)
    declared = _declared_functions()
    assert "load_transformer_ffi" in declared and "yl_forward_x" in declared
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(_lib.EXPORTS) == declared


def test_reference_ffi_signatures(yl):
    from yallma3_mini_inference_amd import transformer
    # lib.rs:138-140: NULL path -> false; unknown extension -> false
    assert transformer.load_transformer_ffi(None) is False
    assert transformer.load_transformer_ffi("/nonexistent/model.bin") is False
    yl.lib().free_string(None)   # NULL-safe


# lib.rs:107-152: the loader is picked by Path::extension of the path, and a
# path that is not UTF-8 is taken as "" (no extension).  Refused paths fail
# before any device or file access; accepted ones fail later (no file here).
@pytest.mark.parametrize("path,accepted", [
    ("m.gguf", True), ("/a/b.c/m.lmrs", True), ("x.tar.safetensors", True),
    ("m.gguf/", True), ("m.gguf/.", True), ("m.gguf//", True),
    ("m.GGUF", False), (".gguf", False), ("/a/.gguf", False), ("m.gguf/..", False),
    ("gguf", False), ("m.", False), ("/a.gguf/m", False), ("", False), ("/", False),
    (b"\xff/m.gguf", False), (b"m\xc3.gguf", False),
])
def test_loader_extension_rule(yl, path, accepted):
    from yallma3_mini_inference_amd import transformer
    assert transformer.load_transformer_ffi(path) is False
    refused = "Unsupported model extension" in transformer.last_error()
    assert refused is not accepted, transformer.last_error()


def test_synthetic_normal_statistics(yl):
    import ctypes as C
    out = np.zeros(200000, np.float32)
    assert yl.lib().yl_synthetic_normal(0, 3, 0, out.size, C.c_float(0.02), out.ctypes.data) == 0
    assert abs(out.mean()) < 2e-4 and abs(out.std() - 0.02) < 2e-4
    # any slice of the stream equals the same elements of the whole stream
    part = np.zeros(1000, np.float32)
    yl.lib().yl_synthetic_normal(0, 3, 5000, part.size, C.c_float(0.02), part.ctypes.data)
    np.testing.assert_array_equal(part, out[5000:6000])
    # kurtosis of a normal is 3
    z = out / out.std()
    assert abs(np.mean(z ** 4) - 3.0) < 0.1


def test_synthetic_gguf_deterministic(yl, tmp_path):
    from yallma3_mini_inference_amd import synth
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    synth.write(a, synth.CONFIGS["tiny"])
    synth.write(b, synth.CONFIGS["tiny"])
    da, db = open(a, "rb").read(), open(b, "rb").read()
    assert da == db
    expect = open(os.path.join(GOLDEN, "tiny_seed0.sha256")).read().split()[0]
    assert hashlib.sha256(da).hexdigest() == expect


@pytest.mark.parametrize("name", ["tiny", "tiny_q4", "tiny_mixed"])
def test_synthetic_gguf_loads_in_oracle(yl, oracle, tmp_path, name):
    from yallma3_mini_inference_amd import synth
    cfg = synth.CONFIGS[name]
    p = synth.write(str(tmp_path / f"{name}.gguf"), cfg)
    m = oracle.Model(p)
    assert (m.dim, m.hidden, m.n_layers, m.n_heads, m.n_kv_heads, m.vocab, m.ctx_len) == (
        cfg.dim, cfg.hidden, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.vocab, cfg.ctx_len)
    emb = m.embedding().reshape(cfg.vocab, cfg.dim)
    assert abs(float(emb.std()) - cfg.weight_std) < 0.1 * cfg.weight_std
    # max_ctx_len caps llama.context_length (gguf.rs:233)
    m2 = oracle.Model(p, max_ctx_len=16)
    assert m2.ctx_len == 16
