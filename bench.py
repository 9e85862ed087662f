"""Decode benchmark: Llama-3.2-1B-shaped Q8_0, batch 1, on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Workload: seeded synthetic Llama-3.2-1B-shaped Q8_0 GGUF (dim 2048, FFN 8192,
16 layers, 32/8 heads, vocab 128256, RoPE theta 500000, tied embedding,
weights ~N(0, 0.02)), KV cache f32 for ctx 4096.  A 512-token random prompt
is prefilled (untimed), then W warmup and K timed greedy decode steps run at
positions 512 .. 512+W+K-1 (default W + K = 256).  A step is one forward_x
of one token plus the device argmax that feeds the next step (one HIP graph
launch; tokens stay on the device).

Also reported (same JSON line):
  kernels       per kernel class (QKV / Wo / gate-up / down GEMV, attention,
                logits): the class's launches of one decode step (one per
                layer) captured back to back in a HIP graph and replayed
                between two HIP events on the session's stream, after the
                timed steps, at the last decoded position; average us per
                launch and algorithmic bytes per launch (quantized weights +
                f16 scales + activations read + outputs written).
  roofline      the dominant kernel (the GEMV class with the most time per
                token): its bytes per launch / its average launch time,
                against 8 TB/s; `traffic` = the HBM bytes per launch measured
                by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, calibrated on a
                copy kernel) from profiles/pmc_traffic_llama32_1b_decode.json
                when that file covers this kernel, else null.
  gemv_all      all four GEMV classes together: weight bytes per token / GEMV
                time per token from the per-class replays.
  in_step       the decode step as its graph launches it, replayed whole and
                without each class's launches (yl_profile_step): a class's
                cost inside the step, kernel boundaries included, is the
                difference; gemv_all over those costs (the 60%-of-8-TB/s
                target's figure inside the step).
  cpu_baseline  the oracle (C restatement of the reference's Rayon CPU path,
                OpenMP) decoding a bounded sample of the same workload on this
                host's cores; `variants` times the same sample at the
                reference's default thread count (ceil(50% of cores)) and as an
                SSE2-only build (the reference's Cargo.toml sets no
                target-cpu), in child processes.
  parity        outside the timed region: the HIP path decodes the same
                sample (same random-filled KV cache, same first token) one
                forward_x at a time, and every step's logits and greedy token
                are compared with the oracle's: bit-identical logits, the
                largest relative logit difference (bar 1e-3) and whether the
                greedy tokens are identical.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s + quant GEMV HBM GB/s (% of 8 TB/s peak), Llama-3.2-1B shape"
HBM_PEAK_GBS = 8000.0
KERNEL_NAMES = {
    "qkv": "k_gemv (QKV, RMSNorm prologue, RoPE/KV epilogue)",
    "wo": "k_gemv (Wo, residual epilogue)",
    "w13": "k_gemv (gate/up, RMSNorm prologue, SwiGLU + quantize epilogue)",
    "w2": "k_gemv (down, residual epilogue)",
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


SAMPLE_STEPS = 64   # decode steps of the CPU-baseline and parity sample


def sample_kv(shape, prompt_len):
    """The sample's KV cache below prompt_len: N(0, 1), seed 0 (keys, values)."""
    import numpy as np
    rng = np.random.default_rng(0)
    kv_dim = shape.n_kv_heads * shape.head_size
    dims = (shape.n_layers, prompt_len, kv_dim)
    return rng.standard_normal(dims, dtype=np.float32), rng.standard_normal(dims, dtype=np.float32)


def gpu_sample(model, kv, prompt_len, attention):
    """The HIP path on the sample: forward_x one token at a time from token 1
    at prompt_len, greedy; returns (per-step logits, tokens)."""
    import numpy as np
    import yallma3_mini_inference_amd as Y
    sess = model.create_session()
    sess.set_attention(attention)
    sess.upload_kv(*kv)
    tok, logits, toks = 1, [], []
    for i in range(SAMPLE_STEPS):
        lg = model.forward_x([tok], prompt_len + i, sess)
        tok = int(np.argmax(lg))
        logits.append(lg)
        toks.append(tok)
    sess.close()
    Y.lib().yl_synchronize()
    return logits, toks


def cpu_baseline(path, prompt_len, seconds, kv):
    """Oracle decode at positions prompt_len.. with the sample's KV cache;
    returns the baseline record and the per-step logits and tokens."""
    import numpy as np
    from oracle import oracle as O
    t0 = time.perf_counter()
    m = oracle_model(path)
    s = m.create_session()
    s.key_cache()[:, :prompt_len] = kv[0]
    s.value_cache()[:, :prompt_len] = kv[1]
    log(f"cpu baseline: oracle load {time.perf_counter() - t0:.1f}s, threads {O.num_threads()}")
    tok, pos, n = 1, prompt_len, 0
    logits, toks = [], []
    t0 = time.perf_counter()
    while True:
        lo = m.forward_x([tok], pos, s)
        tok = O.argmax(lo)
        logits.append(lo)
        toks.append(tok)
        pos += 1
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= SAMPLE_STEPS:
            break
    rec = {"value": n / el, "unit": "tok/s", "cores": O.num_threads(), "kind": "port",
           "sample": f"{n} greedy decode steps at positions {prompt_len}..{prompt_len + n - 1} of the same "
                     f"model, KV cache below {prompt_len} random-filled (N(0,1), seed 0), {el:.1f}s"}
    return rec, logits, toks


def cpu_variant_child(path, prompt_len, seconds):
    """Child process of one CPU-baseline variant: the oracle build and thread
    count come from YL_ORACLE_ISA / OMP_NUM_THREADS; prints one JSON line."""
    from oracle import oracle as O

    class _Shape:
        pass
    m = oracle_model(path)
    sh = _Shape()
    sh.n_kv_heads, sh.head_size, sh.n_layers = m.n_kv_heads, m.head_size, m.n_layers
    kv = sample_kv(sh, prompt_len)
    s = m.create_session()
    s.key_cache()[:, :prompt_len] = kv[0]
    s.value_cache()[:, :prompt_len] = kv[1]
    tok, pos, n, toks = 1, prompt_len, 0, []
    t0 = time.perf_counter()
    while True:
        tok = O.argmax(m.forward_x([tok], pos, s))
        toks.append(tok)
        pos += 1
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= SAMPLE_STEPS:
            break
    print(json.dumps({"value": n / el, "steps": n, "seconds": el, "cores": O.num_threads(), "tokens": toks}))


def cpu_variants(path, prompt_len, seconds, ref_tokens):
    """The reference's own defaults beside the all-cores native-ISA baseline:
    ceil(50% of the cores) threads (parallelism.rs:59-71) and the SSE2-only
    build that its Cargo.toml produces (no target-cpu), each in a child
    process on the same sample; its tokens must equal the main baseline's."""
    import math
    import subprocess
    # the cores this process may use: OpenMP's thread count when set (the
    # host's share), else every core the OS reports
    cores = int(os.environ.get("OMP_NUM_THREADS") or 0) or os.cpu_count() or 1
    half = math.ceil(cores / 2)
    out = []
    for isa, threads, what in (("native", half, "reference default threads ceil(50% of cores), native ISA"),
                               ("sse2", cores, "SSE2-only build (the reference's Cargo.toml), all cores"),
                               ("sse2", half, "SSE2-only build, ceil(50% of cores): the reference's defaults")):
        env = dict(os.environ, OMP_NUM_THREADS=str(threads))
        if isa != "native":
            env["YL_ORACLE_ISA"] = isa
        else:
            env.pop("YL_ORACLE_ISA", None)
        cmd = [sys.executable, os.path.abspath(__file__), "--cpu-variant-child", path, "--prompt", str(prompt_len),
               "--cpu-seconds", str(seconds)]
        res = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=600)
        if res.returncode != 0:
            log(f"cpu variant {what}: failed: {res.stderr[-400:]}")
            continue
        r = json.loads(res.stdout.strip().splitlines()[-1])
        n = r["steps"]
        out.append({"value": round(r["value"], 3), "unit": "tok/s", "cores": r["cores"], "isa": isa,
                    "what": what, "steps": n, "tokens_match": r["tokens"] == list(ref_tokens[:n])})
        log(f"cpu variant {what}: {r['value']:.3f} tok/s on {r['cores']} threads")
    return out


def parity_record(gpu, cpu):
    """Step-by-step comparison of the HIP path's sample with the oracle's."""
    import numpy as np
    (gl, gt), (cl, ct) = gpu, cpu
    n = len(cl)
    worst, bits = 0.0, True
    for a, b in zip(gl[:n], cl):
        a64, b64 = a.astype(np.float64), b.astype(np.float64)
        worst = max(worst, float(np.max(np.abs(a64 - b64)) / max(float(np.max(np.abs(b64))), 1e-30)))
        bits = bits and bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))
    return {"steps_compared": n, "tokens_identical": list(gt[:n]) == list(ct), "logits_bit_identical": bits,
            "max_rel_logit_diff": worst, "tolerance": 1e-3,
            "sample": "the cpu_baseline sample, decoded on the GPU one forward_x per step"}


MFMA_INT8_PEAK_TOPS = 5000.0

# Decode workloads (--config): prompt length, decode steps (warmup + timed),
# and the description that names them in the result line.
DECODE = {
    "llama32_1b": (512, 256, "Llama-3.2-1B-shaped Q8_0 greedy decode, batch 1, 512-token prompt then 256 steps, "
                             "KV f32 ctx 4096"),
    "smollm2_135m": (256, 128, "SmolLM2-135M-shaped Q8_0 greedy decode, batch 1, 256-token prompt then 128 steps"),
    "llama3_8b_mixed": (8192, 256, "Llama-3-8B-shaped decode (Q4_0 FFN, Q8_0 attention/output), batch 1, KV cache "
                                   "prefilled to 8192 positions, then 256 steps"),
    "lmrs_1b": (512, 256, "Llama-3.2-1B-shaped lm.rs model (Q8, f32 scales per group of 32, HF-layout RoPE) greedy "
                          "decode, batch 1, 512-token prompt then 256 steps, KV f32 ctx 4096"),
    "st_q8_1b": (512, 256, "Llama-3.2-1B-shaped safetensors Q8 model (f32 scales per group of 64, HF-layout RoPE) "
                           "greedy decode, batch 1, 512-token prompt then 256 steps, KV f32 ctx 4096"),
    "st_f16_1b": (512, 256, "Llama-3.2-1B-shaped safetensors F16 model (matmul_f32, HF-layout RoPE) greedy decode, "
                            "batch 1, 512-token prompt then 256 steps, KV f32 ctx 4096"),
}

# Models of the lm.rs and safetensors formats (synth_files), and the kernel
# that runs each GEMV class of theirs.
FILE_CONFIGS = {"lmrs_1b", "st_q8_1b", "st_f16_1b"}
FILE_KERNELS = {
    "lmrs_1b": {"qkv": "k_gemv<kQ8S> (q|k|v rows with f32 block scales, q/k heads in RoPE pair order; RMSNorm "
                       "prologue, RoPE + KV-cache epilogue)",
                "wo": "k_gemv<kQ8S> (output projection, residual add)",
                "w13": "k_gemv<kQ8S> (32 gate + 32 up rows per workgroup, RMSNorm prologue, SwiGLU + quantize "
                       "epilogue)", "w2": "k_gemv<kQ8S> (down, residual add)"},
    "st_q8_1b": {"qkv": "k_gemv<kQ8S64> (q|k|v rows, f32 scales per 64-group, q/k heads in RoPE pair order; "
                        "RMSNorm + 64-group quantize prologue, RoPE + KV-cache epilogue)",
                 "wo": "k_gemv<kQ8S64> (output projection; f32 attention row quantized in the prologue, residual add)",
                 "w13": "k_gemv<kQ8S64> (32 gate + 32 up rows per workgroup, RMSNorm prologue, SwiGLU epilogue, "
                        "f32 h)", "w2": "k_gemv<kQ8S64> (down; f32 h quantized in the prologue, residual add)"},
    "st_f16_1b": {"qkv": "k_f16_gemv (fused q/k/v rows, RMSNorm prologue)", "wo": "k_f16_gemv (output, residual add)",
                  "w13": "k_f16_gemv (gate/up row pairs, RMSNorm prologue, SwiGLU epilogue)",
                  "w2": "k_f16_gemv (down, residual add)"},
}


def model_path(config):
    from yallma3_mini_inference_amd import synth, synth_files
    return synth_files.ensure(config) if config in FILE_CONFIGS else synth.ensure(config)


def oracle_model(path):
    """The oracle's model of a GGUF, lm.rs or safetensors file."""
    from oracle import oracle as O
    if path.endswith(".gguf"):
        return O.Model(path)
    from oracle import loaders
    return (loaders.load_lmrs if path.endswith(".lmrs") else loaders.load_safetensors)(path)[0]


def run_prefill(args):
    """Llama-3.2-1B-shaped Q4_0 (Q4_0 activations, reference semantics): a prompt of
    --prefill-tokens random ids in one forward_x (projections on the int8-MFMA
    GEMM), then --steps greedy decode steps.  Per-class GEMM times come from graph
    replays of each projection's 16 launches at the prompt's batch."""
    import numpy as np
    import yallma3_mini_inference_amd as Y
    from yallma3_mini_inference_amd import synth
    M = args.prefill_tokens
    path = synth.ensure("llama32_1b_q4")
    model = Y.Transformer(path)
    sess = model.create_session()
    sh = model.shape
    rng = np.random.default_rng(0)
    prompt = rng.integers(0, model.vocab_size(), M).astype(np.uint32)
    model.forward_argmax(prompt, 0, sess)          # first use: kernel set-up, buffers
    sess.reset()
    Y.lib().yl_synchronize()
    t0 = time.perf_counter()
    first = model.forward_argmax(prompt, 0, sess)
    Y.lib().yl_synchronize()
    pre_s = time.perf_counter() - t0
    log(f"prefill {M} tokens: {pre_s * 1e3:.1f} ms -> {M / pre_s:.0f} tok/s")
    steps = min(args.steps, 256)
    t0 = time.perf_counter()
    toks = model.generate_greedy(sess, first, M, steps)
    Y.lib().yl_synchronize()
    dec_s = time.perf_counter() - t0
    log(f"decode after prefill: {steps} steps in {dec_s * 1e3:.1f} ms -> {steps / dec_s:.1f} tok/s")
    dim, hid, att, kv = sh.dimension, sh.hidden_dimension, sh.n_heads * sh.head_size, sh.n_kv_heads * sh.head_size
    shapes = {"qkv": (att + 2 * kv, dim), "wo": (dim, att), "w13": (2 * hid, dim), "w2": (dim, hid)}
    kern, gemm_us, gemm_ops = {}, 0.0, 0
    for cls in ("qkv", "wo", "w13", "w2", "attention"):
        us, _, n = model.profile_kernel(sess, first, 0, cls, reps=3, batch=M)
        kern[cls] = {"us": round(us, 1), "launches_per_step": n}
        if cls in shapes:
            o, k = shapes[cls]
            ops = 2 * M * o * k
            kern[cls]["tops"] = round(ops / (us * 1e-6) / 1e12, 1)
            gemm_us += us * n
            gemm_ops += ops * n
        log(f"{cls}: {us:.1f} us/launch" + (f" -> {kern[cls]['tops']} TOP/s" if cls in shapes else ""))
    tops = gemm_ops / (gemm_us * 1e-6) / 1e12
    log(f"GEMMs: {gemm_ops / 1e12:.3f} T int8 ops in {gemm_us / 1e3:.2f} ms -> {tops:.0f} TOP/s "
        f"({tops / MFMA_INT8_PEAK_TOPS * 100:.1f}% of {MFMA_INT8_PEAK_TOPS:.0f})")
    print(json.dumps({
        "metric": f"prefill tok/s, Llama-3.2-1B-shaped Q4_0, {M}-token prompt (int8-MFMA GEMM)",
        "value": round(M / pre_s, 1), "unit": "tok/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "int8", "data": "synthetic (seeded N(0,0.02) weights, GGUF Q4_0; random prompt ids)",
        "config": {"workload": f"Llama-3.2-1B-shaped Q4_0 prefill of {M} tokens, then {steps} greedy steps",
                   "prompt_tokens": M},
        "prefill_ms": round(pre_s * 1e3, 2),
        "roofline": {"bound": "mfma", "achieved": round(tops, 1), "peak": MFMA_INT8_PEAK_TOPS, "unit": "TOP/s",
                     "frac": round(tops / MFMA_INT8_PEAK_TOPS, 4), "traffic": None,
                     "kernel": "k_gemm (int8 MFMA, all four projections)",
                     "int_ops_per_prefill": gemm_ops, "gemm_ms": round(gemm_us / 1e3, 3)},
        "kernels": kern,
        "decode_tok_s_after_prefill": round(steps / dec_s, 1),
        "tokens_head": [int(t) for t in toks[:8]],
    }), flush=True)


def run_matvec(args):
    """The isolated Q8_0 matvec: W 8192x2048 ~N(0,0.02) as GGUF Q8_0 blocks, x 2048
    ~N(0,1) quantized Q8_0, out 8192 f32, seed 0; 1000 launches rotating through 24
    device copies of W (408 MiB, beyond the 256 MiB MALL)."""
    import ctypes as C
    import numpy as np
    import yallma3_mini_inference_amd as Y
    from oracle import oracle as O
    L = Y.lib()
    o, n, copies, iters = 8192, 2048, 24, 1000
    wf = np.zeros(o * n, np.float32)
    xf = np.zeros(n, np.float32)
    Y.check(L.yl_synthetic_normal(0, 0, 0, wf.size, C.c_float(0.02), wf.ctypes.data))
    Y.check(L.yl_synthetic_normal(0, 1, 0, xf.size, C.c_float(1.0), xf.ctypes.data))
    blocks = wf.reshape(-1, 32)
    d = (np.abs(blocks).max(axis=1) / np.float32(127.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), 0).astype(np.float32)
    q = np.round(blocks * inv[:, None]).astype(np.int8)
    raw = np.zeros((blocks.shape[0], 34), np.uint8)
    raw[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    raw[:, 2:] = q.view(np.uint8)
    ws = [Y.QuantizedWeight.upload_gguf(Y.WeightFormat.Q8_0, raw.ravel(), o, n) for _ in range(copies)]
    xq, xs = Y.quantize(Y.WeightFormat.Q8_0, xf)
    dq, ds = Y.DeviceBuffer.from_numpy(xq), Y.DeviceBuffer.from_numpy(xs)
    dout = Y.DeviceBuffer.from_numpy(np.zeros(o, np.float32))
    handles = (C.c_void_p * copies)(*[w._h for w in ws])
    us = C.c_double()
    Y.check(L.yl_matmul_bench(handles, copies, dq.ptr, ds.ptr, 1, dout.ptr, max(1, iters // copies), C.byref(us)))
    nbytes = o * n + (o * n // 32) * 2 + n + (n // 32) * 4 + o * 4
    gbs = nbytes / (us.value * 1e-6) / 1e9
    # parity of the last launch against the oracle
    out = dout.numpy()
    ref = O.matmul_q8_slices(np.zeros(o, np.float32), xq, xs, q.ravel(),
                             d.astype(np.float16).astype(np.float32), n, o)
    same = bool((out.view(np.uint32) == ref.view(np.uint32)).all())
    log(f"matvec 8192x2048 Q8_0: {us.value:.2f} us/launch, {nbytes} B -> {gbs:.0f} GB/s; bit-exact: {same}")
    t0, k = time.perf_counter(), 0
    while time.perf_counter() - t0 < min(args.cpu_seconds, 10.0) and k < iters:
        O.matmul_q8_slices(np.zeros(o, np.float32), xq, xs, q.ravel(), d.astype(np.float16).astype(np.float32), n, o)
        k += 1
    cpu_us = (time.perf_counter() - t0) / k * 1e6
    print(json.dumps({
        "metric": "isolated Q8_0 matvec 8192x2048 GB/s", "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
        "higher_is_better": True, "dtype": "int8", "data": "synthetic (seed 0, W ~N(0,0.02) GGUF Q8_0, x ~N(0,1))",
        "config": {"workload": f"8192x2048 Q8_0 matvec, {iters} launches over {copies} weight copies"},
        "us_per_launch": round(us.value, 3), "bit_exact": same,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "k_gemv (store epilogue)", "bytes_per_launch": nbytes},
        "cpu_baseline": {"value": round(cpu_us, 1), "unit": "us/matvec", "cores": O.num_threads(), "kind": "port",
                         "sample": f"{k} oracle matmul_q8_slices calls on the same inputs"},
    }), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed decode steps (default: the workload's steps - warmup)")
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=None, help="prompt tokens (default: the workload's)")
    ap.add_argument("--config", default="llama32_1b", choices=sorted(DECODE),
                    help="decode workload: llama32_1b (the headline), smollm2_135m, llama3_8b_mixed, lmrs_1b "
                         "(lm.rs Q8 with f32 scales per 32), st_q8_1b (safetensors Q8 with f32 scales per 64), "
                         "st_f16_1b (safetensors F16)")
    ap.add_argument("--attention", choices=("exact", "split"), default="exact",
                    help="decode attention: exact (the reference's operation order, bit-exact; the default) or "
                         "split over the context (equal up to rounding; on these synthetic models rounding-level "
                         "differences can move the logits by more than 1e-3 at some steps)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=("decode", "prefill", "matvec"), default="decode",
                    help="decode: the headline Llama-3.2-1B Q8_0 decode (default); prefill: Llama-3.2-1B Q4_0 "
                         "prompt of --prefill-tokens on the int8-MFMA GEMM, then greedy decode; matvec: the "
                         "isolated 8192x2048 Q8_0 matvec")
    ap.add_argument("--prefill-tokens", type=int, default=2048)
    ap.add_argument("--cpu-variants", action=argparse.BooleanOptionalAction, default=True,
                    help="also time the oracle at the reference's default thread count and as an SSE2-only build")
    ap.add_argument("--cpu-variant-child", default=None, help=argparse.SUPPRESS)
    ap.add_argument("--stream-table", action="store_true",
                    help="also print a markdown table: each GEMV class's graph replay against a plain stream of "
                         "its own weight bytes with the same grid (GGUF configs)")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="first run one plain device copy of this many MiB (the known-size kernel that "
                         "calibrates rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.cpu_variant_child:   # oracle only: no GPU in this process
        return cpu_variant_child(args.cpu_variant_child, args.prompt, args.cpu_seconds)
    if args.gpus != 1:
        print(f"bench.py runs on one GPU; --gpus {args.gpus} is not supported (the decode path is "
              f"single-GPU, see DESIGN.md for how it would shard)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import yallma3_mini_inference_amd as Y
    from yallma3_mini_inference_amd import synth

    if Y.device_count() < 1:
        print("no HIP device visible", file=sys.stderr)
        sys.exit(1)
    if args.calibrate_copy_mib:
        # the runtime's plain copy kernel over a known number of bytes
        nbytes = args.calibrate_copy_mib << 20
        L = Y.lib()
        src, dst = L.yl_malloc(nbytes), L.yl_malloc(nbytes)
        if not src or not dst:
            raise SystemExit("calibration buffers: allocation failed")
        Y.check(L.yl_memset_d(src, 1, nbytes))
        Y.check(L.yl_memcpy_d2d(dst, src, nbytes))
        Y.check(L.yl_synchronize())
        L.yl_free(src)
        L.yl_free(dst)
        log(f"calibration copy: {nbytes} B read + {nbytes} B written")
    if args.workload == "prefill":
        if args.steps is None:
            args.steps = 32
        return run_prefill(args)
    if args.workload == "matvec":
        return run_matvec(args)
    d_prompt, d_steps, d_desc = DECODE[args.config]
    if args.prompt is None:
        args.prompt = d_prompt
    if args.steps is None:
        args.steps = d_steps - args.warmup
    t0 = time.perf_counter()
    path = model_path(args.config)
    log(f"model {path} ready in {time.perf_counter() - t0:.1f}s")
    t0 = time.perf_counter()
    model = Y.Transformer(path)
    sess = model.create_session()
    attention = args.attention
    sess.set_attention(attention)
    log(f"decode attention: {attention}")
    log(f"loaded to HBM in {time.perf_counter() - t0:.1f}s; GEMV weights {model.weight_bytes()} B/token, "
        f"logits embedding {model.embedding_bytes()} B/token")
    ctx = model.max_ctx_len()
    if args.prompt + args.warmup + args.steps > ctx:
        print("prompt + warmup + steps exceed the context", file=sys.stderr)
        sys.exit(2)

    rng = np.random.default_rng(0)
    prompt = rng.integers(0, model.vocab_size(), args.prompt).astype(np.uint32)
    t0 = time.perf_counter()
    first = model.forward_argmax(prompt, 0, sess)
    Y.lib().yl_synchronize()
    prefill_s = time.perf_counter() - t0
    log(f"prefill {args.prompt} tokens: {prefill_s * 1e3:.1f} ms")

    pos = args.prompt
    warm = model.generate_greedy(sess, first, pos, args.warmup) if args.warmup else np.array([first], np.uint32)
    pos += args.warmup
    nxt = int(warm[-1])
    Y.lib().yl_synchronize()
    t0 = time.perf_counter()
    toks = model.generate_greedy(sess, nxt, pos, args.steps)
    Y.lib().yl_synchronize()
    elapsed = time.perf_counter() - t0
    tok_s = args.steps / elapsed
    log(f"decode: {args.steps} steps in {elapsed * 1e3:.1f} ms -> {tok_s:.1f} tok/s")

    # per-class kernel timing: each class's launches of one decode step replayed
    # as a graph between two HIP events on the session's stream (at the last
    # decoded position; this modifies the session, which is not used again)
    ppos = pos + args.steps - 1
    kern = {}
    for cls, reps in (("qkv", 20), ("attention", 20), ("wo", 20), ("w13", 20), ("w2", 20), ("logits", 10)):
        us, nb, n = model.profile_kernel(sess, nxt, ppos, cls, reps)
        kern[cls] = {"us": round(us, 3), "bytes": int(nb), "launches_per_step": int(n)}
        if nb:
            kern[cls]["gbs"] = round(nb / (us * 1e-6) / 1e9, 1)
        log(f"{cls}: {us:.2f} us/launch x {n}/step" + (f", {nb / 1e6:.2f} MB -> {nb / (us * 1e3):.0f} GB/s" if nb else ""))
    if args.stream_table and args.config not in FILE_CONFIGS:
        print("| class | bytes per launch | GEMV us (replay) | plain stream us | GEMV TB/s | stream TB/s | "
              "GEMV / stream |", file=sys.stderr)
        print("|---|---|---|---|---|---|---|", file=sys.stderr)
        for cls in ("qkv", "wo", "w13", "w2"):
            sus, sb = model.profile_stream(sess, cls, reps=20)
            gus = kern[cls]["us"]
            print(f"| {cls} | {sb:,} | {gus:.2f} | {sus:.2f} | {sb / gus / 1e6:.2f} | {sb / sus / 1e6:.2f} | "
                  f"{gus / sus:.2f} |", file=sys.stderr, flush=True)
    # the step as its graph launches it, whole and without each class
    step_us = model.profile_step(sess, nxt, ppos, None, reps=20)
    marg = {}
    for cls in ("qkv", "attention", "wo", "w13", "w2", "logits"):
        marg[cls] = round(step_us - model.profile_step(sess, nxt, ppos, cls, reps=20), 2)
    log(f"step replay {step_us:.1f} us; cost of each class inside it: " +
        ", ".join(f"{c} {v:.1f}" for c, v in marg.items()))
    gemv = ("qkv", "wo", "w13", "w2")
    gemv_us = sum(kern[c]["us"] * kern[c]["launches_per_step"] for c in gemv)
    gemv_bytes = sum(kern[c]["bytes"] * kern[c]["launches_per_step"] for c in gemv)
    gemv_gbs = gemv_bytes / (gemv_us * 1e-6) / 1e9
    log(f"GEMVs: {gemv_us:.1f} us/token for {gemv_bytes / 1e6:.1f} MB -> {gemv_gbs:.0f} GB/s "
        f"({gemv_gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)")
    gemv_in = sum(marg[c] for c in gemv)
    gemv_in_gbs = gemv_bytes / (gemv_in * 1e-6) / 1e9 if gemv_in > 0 else 0.0
    log(f"GEMVs inside the step: {gemv_in:.1f} us/token -> {gemv_in_gbs:.0f} GB/s "
        f"({gemv_in_gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)")
    dom = max(gemv, key=lambda c: kern[c]["us"] * kern[c]["launches_per_step"])
    dom_gbs = kern[dom]["bytes"] / (kern[dom]["us"] * 1e-6) / 1e9
    traffic = None
    tf = os.path.join(ROOT, "profiles", "pmc_traffic_llama32_1b_decode.json")
    if args.config == "llama32_1b" and os.path.exists(tf):
        with open(tf) as f:
            t = json.load(f)
        if t.get("class") == dom:
            traffic = t.get("traffic_bytes_per_launch")

    result = {
        "metric": METRIC if args.config == "llama32_1b" else f"decode tok/s, {args.config} shape",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 weights, f32 activations" if args.config == "st_f16_1b" else "int8",
        "data": ("synthetic (seeded N(0,0.02) weights, GGUF blocks; random prompt ids)" if args.config not in
                 FILE_CONFIGS else "synthetic (seeded random weights, lm.rs / safetensors file; random prompt ids)"),
        "config": {
            "workload": d_desc,
            "batch": 1, "prompt_tokens": args.prompt,
            "decode_positions": f"{args.prompt + args.warmup}..{args.prompt + args.warmup + args.steps - 1}",
            "parallelism": "single GPU",
            "attention": ("exact (the reference's operation order)" if attention == "exact" else
                          "split over the context (f32 combine)"),
        },
        "roofline": {
            "bound": "hbm", "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": FILE_KERNELS.get(args.config, KERNEL_NAMES)[dom], "class": dom,
            "avg_launch_us": kern[dom]["us"], "bytes_per_launch": kern[dom]["bytes"],
        },
        "gemv_all": {"us_per_token": round(gemv_us, 2), "bytes_per_token": gemv_bytes,
                     "achieved_gbs": round(gemv_gbs, 1), "frac": round(gemv_gbs / HBM_PEAK_GBS, 4),
                     "from": "per-class graph replays"},
        "in_step": {"step_replay_us": round(step_us, 2), "class_cost_us_per_step": marg,
                    "gemv_all": {"us_per_token": round(gemv_in, 2), "bytes_per_token": gemv_bytes,
                                 "achieved_gbs": round(gemv_in_gbs, 1),
                                 "frac": round(gemv_in_gbs / HBM_PEAK_GBS, 4)},
                    "how": "decode step graph replayed whole and without each class's launches; a class's "
                           "cost = difference (its kernels and the boundaries they bring)"},
        "kernels": kern,
        "prefill_ms": round(prefill_s * 1e3, 2),
        "tokens_head": [int(t) for t in toks[:8]],
    }
    if not args.no_cpu_baseline:
        sess.close()
        kv = sample_kv(model.shape, args.prompt)
        gpu = gpu_sample(model, kv, args.prompt, attention)
        model.close()
        rec, cl, ct = cpu_baseline(path, args.prompt, args.cpu_seconds, kv)
        result["cpu_baseline"] = rec
        result["parity"] = parity_record(gpu, (cl, ct))
        log(f"cpu baseline {rec['value']:.3f} tok/s; parity {result['parity']}")
        if args.cpu_variants:
            rec["variants"] = cpu_variants(path, args.prompt, min(args.cpu_seconds, 10.0), ct)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
