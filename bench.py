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
  roofline      the quantized GEMV kernels (all seven projections): their
                algorithmic bytes (quantized weights + f16 scales + int8
                activations + outputs) / their HIP-event time, measured on
                the session's stream over P decode steps run eagerly with an
                event pair around every GEMV launch, against 8 TB/s.
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
    ap.add_argument("--profile-steps", type=int, default=32)
    ap.add_argument("--config", default="llama32_1b")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
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

    # roofline of the quantized GEMV kernels (event pairs around every launch)
    ms, launches, nbytes = model.profile_decode(sess, nxt, args.prompt, args.profile_steps, 0)
    gemv_gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"GEMV: {launches} launches, {nbytes / launches / 1e6:.2f} MB avg, {ms / launches * 1e3:.2f} us avg "
        f"-> {gemv_gbs:.0f} GB/s")
    a_ms, a_n, _ = model.profile_decode(sess, nxt, args.prompt, 8, 1)
    l_ms, l_n, l_bytes = model.profile_decode(sess, nxt, args.prompt, 8, 2)
    log(f"attention avg {a_ms / a_n * 1e3:.2f} us; logits avg {l_ms / l_n * 1e3:.2f} us "
        f"({l_bytes / (l_ms * 1e-3) / 1e9:.0f} GB/s)")

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
            "bound": "hbm", "achieved": round(gemv_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gemv_gbs / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "k_gemv (quantized GEMV, all projections)",
            "avg_launch_us": round(ms / launches * 1e3, 3), "bytes_per_launch": int(nbytes // launches),
        },
        "prefill_ms": round(prefill_s * 1e3, 2),
        "attention_avg_us": round(a_ms / a_n * 1e3, 3),
        "logits_avg_us": round(l_ms / l_n * 1e3, 3),
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
