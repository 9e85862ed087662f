"""Builds libyallma3_amd.so in-tree with hipcc for gfx950.

    python -m yallma3_mini_inference_amd.build      (or build() from Python)

Every HIP source is compiled with -ffp-contract=off (no fused multiply-add:
the forward path reproduces the reference's separately rounded f32 products
and sums) and with packed FP32 instructions disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB_DIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIB_DIR, "libyallma3_amd.so")

SOURCES = ["yl_kernels.hip", "yl_gemv.hip", "yl_gemm.hip", "yl_attn.hip", "yl_attn_split.hip", "yl_pattn.hip", "yl_logits.hip", "yl_f16.hip", "yl_q8g.hip", "yl_model.hip",
           "yl_gguf.cpp", "yl_synth.cpp", "yl_tokenizer.cpp", "yl_jinja.cpp", "yl_loaders.cpp"]
ARCH = os.environ.get("YL_OFFLOAD_ARCH", "gfx950")

COMMON = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", "-Wno-unused-function",
          "-Wno-unused-variable", "-Wno-unused-result", "-Wno-unused-value", f"-I{os.path.join(os.path.dirname(PKG), 'include')}"]
HIP_ONLY = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP extension)")


def _compile(src: str) -> str:
    os.makedirs(OBJ, exist_ok=True)
    path = os.path.join(CSRC, src)
    obj = os.path.join(OBJ, src + ".o")
    if src.endswith(".hip"):
        cmd = [_hipcc(), *COMMON, *HIP_ONLY, "-c", path, "-o", obj]
    else:
        cmd = [_hipcc(), *COMMON, "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-x", "c++", "-c", path,
               "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{msgs}")
    if msgs.strip():
        print(msgs, file=sys.stderr)
    return obj


def build(verbose: bool = False) -> str:
    """Compile every source and link the shared library; returns its path."""
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
