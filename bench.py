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
                time per token (the 60%-of-8-TB/s target's figure).
  cpu_baseline  the oracle (C restatement of the reference's Rayon CPU path,
                OpenMP) decoding a bounded sample of the same workload on this
                host's cores.
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


def cpu_baseline(path, prompt_len, seconds):
    """Oracle decode at positions prompt_len.. with a random-filled KV cache."""
    import numpy as np
    from oracle import oracle as O
    t0 = time.perf_counter()
    m = O.Model(path)
    s = m.create_session()
    rng = np.random.default_rng(0)
    kc, vc = s.key_cache(), s.value_cache()
    kc[:, :prompt_len] = rng.normal(0, 1, kc[:, :prompt_len].shape).astype(np.float32)
    vc[:, :prompt_len] = rng.normal(0, 1, vc[:, :prompt_len].shape).astype(np.float32)
    log(f"cpu baseline: oracle load {time.perf_counter() - t0:.1f}s, threads {O.num_threads()}")
    tok, pos, n = 1, prompt_len, 0
    t0 = time.perf_counter()
    while True:
        tok = O.argmax(m.forward_x([tok], pos, s))
        pos += 1
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 64:
            break
    return {"value": n / el, "unit": "tok/s", "cores": O.num_threads(), "kind": "port",
            "sample": f"{n} greedy decode steps at positions {prompt_len}..{prompt_len + n - 1} of the same "
                      f"model, KV cache below {prompt_len} random-filled, {el:.1f}s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--config", default="llama32_1b")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="first run one plain device copy of this many MiB (the known-size kernel that "
                         "calibrates rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
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
    t0 = time.perf_counter()
    path = synth.ensure(args.config)
    log(f"model {path} ready in {time.perf_counter() - t0:.1f}s")
    t0 = time.perf_counter()
    model = Y.Transformer(path)
    sess = model.create_session()
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
    gemv = ("qkv", "wo", "w13", "w2")
    gemv_us = sum(kern[c]["us"] * kern[c]["launches_per_step"] for c in gemv)
    gemv_bytes = sum(kern[c]["bytes"] * kern[c]["launches_per_step"] for c in gemv)
    gemv_gbs = gemv_bytes / (gemv_us * 1e-6) / 1e9
    log(f"GEMVs: {gemv_us:.1f} us/token for {gemv_bytes / 1e6:.1f} MB -> {gemv_gbs:.0f} GB/s "
        f"({gemv_gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)")
    dom = max(gemv, key=lambda c: kern[c]["us"] * kern[c]["launches_per_step"])
    dom_gbs = kern[dom]["bytes"] / (kern[dom]["us"] * 1e-6) / 1e9
    traffic = None
    tf = os.path.join(ROOT, "profiles", "pmc_traffic_llama32_1b_decode.json")
    if os.path.exists(tf):
        with open(tf) as f:
            t = json.load(f)
        if t.get("class") == dom:
            traffic = t.get("traffic_bytes_per_launch")

    result = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights, GGUF Q8_0; random prompt ids)",
        "config": {
            "workload": "Llama-3.2-1B-shaped Q8_0 greedy decode, batch 1, 512-token prompt then 256 steps, "
                        "KV f32 ctx 4096",
            "batch": 1, "prompt_tokens": args.prompt,
            "decode_positions": f"{args.prompt + args.warmup}..{args.prompt + args.warmup + args.steps - 1}",
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm", "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": KERNEL_NAMES[dom], "class": dom,
            "avg_launch_us": kern[dom]["us"], "bytes_per_launch": kern[dom]["bytes"],
        },
        "gemv_all": {"us_per_token": round(gemv_us, 2), "bytes_per_token": gemv_bytes,
                     "achieved_gbs": round(gemv_gbs, 1), "frac": round(gemv_gbs / HBM_PEAK_GBS, 4)},
        "kernels": kern,
        "prefill_ms": round(prefill_s * 1e3, 2),
        "tokens_head": [int(t) for t in toks[:8]],
    }
    if not args.no_cpu_baseline:
        sess.close()
        model.close()
        result["cpu_baseline"] = cpu_baseline(path, args.prompt, args.cpu_seconds)
        log(f"cpu baseline {result['cpu_baseline']['value']:.3f} tok/s")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
