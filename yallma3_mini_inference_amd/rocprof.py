"""Summaries of rocprofv3 output for the decode benchmark.

    python -m yallma3_mini_inference_amd.rocprof trace KERNEL_TRACE.csv > summary.md
        Per kernel (name, grid): dispatch count, mean / median / min duration
        (us).  Decode launches (grid y = 1) and prompt launches (grid y > 1,
        one row per token, and the prompt attention kernels) are listed apart, since the bench's per-launch
        figures are for decode launches only.

    python -m yallma3_mini_inference_amd.rocprof instep KERNEL_TRACE.csv N_LAYERS
        The decode steps inside the trace (runs of 5 kernels per layer and the
        logits kernel, as one decode graph launches them): per kernel class,
        the mean duration within the steps, the mean gap between a kernel's
        end and the next one's start, and the step's span (first start to
        last end) -- the in-graph figures, as opposed to per-class replays.

    python -m yallma3_mini_inference_amd.rocprof pmc FETCH.csv WRITE.csv MIB CLASS OUT.json
        HBM bytes per launch of one GEMV class from the counter_collection.csv
        files of `rocprofv3 --pmc FETCH_SIZE` and `rocprofv3 --pmc WRITE_SIZE`
        runs of `bench.py --calibrate-copy-mib MIB`.  Both counters are KiB per
        dispatch; the plain copy of MIB MiB (the largest dispatch whose name
        contains "copy" or "elementwise") scales each counter to real bytes.
        Writes the median scaled FETCH + WRITE bytes per decode dispatch (the
        class's dispatches with the smallest grid).

    python -m yallma3_mini_inference_amd.rocprof pmctable FETCH.csv WRITE.csv MIB
        The same per launch for every class of CLASS_KERNELS (the four GEMVs
        and the decode attention), as a markdown table against the algorithmic
        bytes the bench counts (ALGO_BYTES).

    python -m yallma3_mini_inference_amd.rocprof sq COUNTERS.csv KERNEL_TRACE.csv
        Per decode kernel class, medians over its decode dispatches of the SQ
        counters of one `rocprofv3 --pmc SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES
        SQ_WAIT_INST_ANY SQ_INSTS_VALU SQ_INSTS_LDS` run (summed over the
        XCDs), with the share of wave cycles spent waiting on an instruction's
        operands (SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES) and the duration from the
        kernel trace of the same run.

    python -m yallma3_mini_inference_amd.rocprof mfma COUNTERS.csv KERNEL_TRACE.csv PATTERN
        MFMA utilisation of the kernels whose name contains PATTERN, from one
        `rocprofv3 --kernel-trace --pmc SQ_VALU_MFMA_BUSY_CYCLES
        SQ_INSTS_VALU_MFMA_MOPS_I8 GRBM_GUI_ACTIVE` run: per kernel and grid,
        the dispatches' MFMA-busy share of the SIMD cycles (busy cycles summed
        over the SIMDs / (GUI-active cycles of one XCD x 1024 SIMDs),
        rocprofv3's MfmaUtil), the int8 MFMA operations (MOPS_I8 x 512) and those
        operations per second of dispatch time, against the 5.0 POP/s dense
        int8 peak.
"""
import csv
import collections
import json
import statistics
import sys

# template signatures of the decode GEMV kernels at the Llama-3.2-1B shape
# (weight format, epilogue, embedding prologue, lanes per row, slots)
CLASS_KERNELS = {
    "qkv": "k_gemv<0, 1, false, 16, 4>",
    "wo": "k_gemv<0, 2, false, 16, 4>",
    "w13": "k_gemv<0, 3, false, 8, 8>",
    "w2": "k_gemv<0, 2, false, 64, 4>",
    "attention": "k_attn_decode<0, 64, false>",
}
# algorithmic bytes per launch at the Llama-3.2-1B shape, as bench.py counts
# them: quantized weights + f16 scales + activation row read + outputs
# written; attention: K and V rows of one layer at seq_len positions
# (2 * seq * 512 * 4 B) + the query row + the quantized output
ALGO_BYTES = {"qkv": 6699264, "wo": 4466944, "w13": 35663104, "w2": 17843200}


def attention_bytes(seq):
    return 2 * seq * 512 * 4 + 2048 * 4 + 2048 + 2048 // 8


def _short(name):
    name = name.replace("void ", "").replace("yl::", "")
    return name.split("(")[0]


def trace(path):
    rows = list(csv.DictReader(open(path)))
    by = collections.defaultdict(list)
    for r in rows:
        name = r["Kernel_Name"]
        # (the prompt attention kernels run for prompts only, whatever their grid)
        kind = ("prompt" if "k_pattn_" in name else
                "decode" if r["Grid_Size_Y"] == "1" or "attn_decode" in name or "k_attn_scores" in name or "k_attn_pv_j" in name
                else "prompt")
        key = (kind, _short(r["Kernel_Name"]), r["Grid_Size_X"], r["Grid_Size_Y"], r["Workgroup_Size_X"],
               r["VGPR_Count"], r["LDS_Block_Size"], r["Scratch_Size"])
        by[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    print("| launches | kernel | grid (x, y) | threads | VGPRs | LDS B | scratch | mean us | median us | min us | total us |")
    print("|---|---|---|---|---|---|---|---|---|---|---|")
    for kind in ("decode", "prompt"):
        items = [(k, v) for k, v in by.items() if k[0] == kind]
        items.sort(key=lambda kv: -sum(kv[1]))
        for k, v in items:
            print(f"| {len(v)} {kind} | `{k[1]}` | {k[2]}, {k[3]} | {k[4]} | {k[5]} | {k[6]} | {k[7]} | "
                  f"{statistics.mean(v):.2f} | {statistics.median(v):.2f} | {min(v):.2f} | {sum(v):.0f} |")


STEP_CLASSES = ("qkv", "attention", "wo", "w13", "w2")


def instep(path, n_layers):
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    ks = [(_short(r["Kernel_Name"]), int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in rows]
    per_step = 5 * n_layers + 1
    steps = []
    for i, k in enumerate(ks):
        # a decode step: per_step kernels ending in the logits kernel, whose
        # first kernel is a GEMV (QKV with the embedding prologue in layer 0)
        if not k[0].startswith("k_logits") or i + 1 < per_step:
            continue
        seg = ks[i + 1 - per_step:i + 1]
        if not seg[0][0].startswith("k_gemv") or any(x[0].startswith("k_logits") for x in seg[:-1]):
            continue
        steps.append(seg)
    if not steps:
        raise SystemExit("no decode steps found")
    dur = collections.defaultdict(list)
    gaps = []
    spans = []
    for seg in steps:
        spans.append((seg[-1][2] - seg[0][1]) / 1e3)
        for j, (n, a, b) in enumerate(seg):
            cls = "logits" if j == len(seg) - 1 else STEP_CLASSES[j % 5]
            dur[cls].append((b - a) / 1e3)
            if j:
                gaps.append((a - seg[j - 1][2]) / 1e3)
    print(f"{len(steps)} decode steps of {per_step} kernels; step span (first start to last end): "
          f"mean {statistics.mean(spans):.1f} us, median {statistics.median(spans):.1f} us")
    print(f"gap from a kernel's end to the next one's start: mean {statistics.mean(gaps):.2f} us, "
          f"median {statistics.median(gaps):.2f} us")
    print("| class | launches per step | mean us in the step | us per step |")
    print("|---|---|---|---|")
    for cls in STEP_CLASSES + ("logits",):
        v = dur[cls]
        n = 1 if cls == "logits" else n_layers
        print(f"| {cls} | {n} | {statistics.mean(v):.2f} | {statistics.mean(v) * n:.1f} |")


def _per_dispatch(path, counter):
    out = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if r.get("Counter_Name") != counter:
                continue
            d = r["Dispatch_Id"]
            grid = int(r.get("Grid_Size", "0"))
            prev = out.get(d)
            out[d] = (r["Kernel_Name"], float(r["Counter_Value"]) + (prev[1] if prev else 0.0), grid)
    return out


def _scaled(path, counter, calib_bytes, pattern):
    rows = _per_dispatch(path, counter)
    copies = [v for n, v, _ in rows.values() if "copy" in n.lower() or "elementwise" in n.lower()]
    if not copies:
        raise SystemExit(f"{path}: no copy kernel for calibration")
    factor = calib_bytes / (max(copies) * 1024.0)
    match = [(v, g) for n, v, g in rows.values() if pattern in n]
    if not match:
        raise SystemExit(f"{path}: no dispatch matching {pattern!r}")
    # decode launches have the smallest grid (prompt launches add one row of
    # workgroups per token)
    gmin = min(g for _, g in match)
    vals = [v * 1024.0 * factor for v, g in match if g == gmin]
    return statistics.median(vals), factor, len(vals)


def pmc(fetch_csv, write_csv, mib, cls, out):
    pat = CLASS_KERNELS[cls]
    calib = mib * 1024 * 1024
    fb, ff, nf = _scaled(fetch_csv, "FETCH_SIZE", calib, pat)
    wb, wf, nw = _scaled(write_csv, "WRITE_SIZE", calib, pat)
    res = {"class": cls, "kernel_pattern": pat, "fetch_bytes_per_launch": int(fb),
           "write_bytes_per_launch": int(wb), "traffic_bytes_per_launch": int(fb + wb),
           "fetch_scale": round(ff, 4), "write_scale": round(wf, 4), "dispatches": [nf, nw],
           "calibration": f"plain device copy of {mib} MiB (reads {calib} B, writes {calib} B)"}
    with open(out, "w") as f:
        json.dump(res, f, indent=1)
    print(json.dumps(res))


def pmctable(fetch_csv, write_csv, mib, seq=None):
    calib = mib * 1024 * 1024
    print("| class | kernel | algorithmic B/launch | FETCH B/launch (scaled) | WRITE B/launch | traffic / algorithmic |")
    print("|---|---|---|---|---|---|")
    for cls, pat in CLASS_KERNELS.items():
        fb, ff, nf = _scaled(fetch_csv, "FETCH_SIZE", calib, pat)
        wb, wf, nw = _scaled(write_csv, "WRITE_SIZE", calib, pat)
        algo = ALGO_BYTES.get(cls) or (attention_bytes(seq) if seq else 0)
        ratio = f"{(fb + wb) / algo:.3f}" if algo else "-"
        print(f"| {cls} | `{pat}` | {algo:,} | {int(fb):,} | {int(wb):,} | {ratio} |")
    print(f"\nscales: FETCH x{ff:.4f}, WRITE x{wf:.4f}; decode dispatches per class: {nf}, {nw}")


SQ_COUNTERS = ("SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAIT_INST_ANY", "SQ_INSTS_VALU", "SQ_INSTS_LDS")


def sq(counter_csv, trace_csv):
    dur = {}
    with open(trace_csv) as f:
        for r in csv.DictReader(f):
            dur[r["Dispatch_Id"]] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    cnt = _counters(counter_csv)
    print("| class | kernel | dispatches | mean us | " + " | ".join(SQ_COUNTERS) + " | wait / wave cycles |")
    print("|---|---|---|---|" + "---|" * len(SQ_COUNTERS) + "---|")
    for cls, pat in CLASS_KERNELS.items():
        rows = [(d, cs) for d, (n, cs) in cnt.items() if pat in n]
        if not rows:
            continue
        # decode launches: one row of workgroups (grid y = 1) -- the smallest
        # wave count of the class
        waves = {d: sum(cs.get("SQ_WAVES", [0.0])) for d, cs in rows}
        wmin = min(waves.values())
        rows = [(d, cs) for d, cs in rows if waves[d] == wmin]
        med = {c: statistics.median(sum(cs.get(c, [0.0])) for _, cs in rows) for c in SQ_COUNTERS}
        us = [dur[d] for d, _ in rows if d in dur]
        wait = med["SQ_WAIT_INST_ANY"] / med["SQ_WAVE_CYCLES"] if med["SQ_WAVE_CYCLES"] else 0.0
        print(f"| {cls} | `{pat}` | {len(rows)} | {statistics.mean(us) if us else 0:.2f} | " +
              " | ".join(f"{med[c]:.4g}" for c in SQ_COUNTERS) + f" | {wait:.2f} |")


def _counters(path):
    """{dispatch id: (kernel name, {counter: [values over dimensions]})}"""
    out = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            d = r["Dispatch_Id"]
            name, cs = out.setdefault(d, (r["Kernel_Name"], collections.defaultdict(list)))
            cs[r["Counter_Name"]].append(float(r["Counter_Value"]))
    return out


SIMDS = 1024            # 256 CUs x 4 SIMDs
XCDS = 8
INT8_PEAK = 5.0e15      # dense int8 MFMA operations per second


def mfma(counter_csv, trace_csv, pattern):
    dur = {}
    with open(trace_csv) as f:
        for r in csv.DictReader(f):
            dur[r["Dispatch_Id"]] = ((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9,
                                     r["Grid_Size_X"], r["Grid_Size_Y"])
    by = collections.defaultdict(list)
    for d, (name, cs) in _counters(counter_csv).items():
        if pattern not in name or d not in dur:
            continue
        busy = sum(cs.get("SQ_VALU_MFMA_BUSY_CYCLES", [0.0]))
        # rocprofv3 reports GRBM_GUI_ACTIVE summed over the XCDs
        gui = sum(cs.get("GRBM_GUI_ACTIVE", [0.0])) / XCDS
        ops = sum(cs.get("SQ_INSTS_VALU_MFMA_MOPS_I8", [0.0])) * 512.0
        t, gx, gy = dur[d]
        by[(_short(name), gx, gy)].append((busy / (gui * SIMDS) * 100.0 if gui else 0.0, ops, t))
    print("| dispatches | kernel | grid (x, y) | MFMA busy % (median) | int8 MFMA ops / dispatch | mean us "
          "| int8 TOP/s | % of 5.0 POP/s |")
    print("|---|---|---|---|---|---|---|---|")
    for k, v in sorted(by.items(), key=lambda kv: -sum(x[2] for x in kv[1])):
        util = statistics.median(x[0] for x in v)
        ops = statistics.median(x[1] for x in v)
        t = statistics.mean(x[2] for x in v)
        rate = ops / t if t else 0.0
        print(f"| {len(v)} | `{k[0]}` | {k[1]}, {k[2]} | {util:.1f} | {ops:.4g} | {t * 1e6:.1f} | "
              f"{rate / 1e12:.1f} | {100.0 * rate / INT8_PEAK:.2f} |")


if __name__ == "__main__":
    if len(sys.argv) >= 3 and sys.argv[1] == "trace":
        trace(sys.argv[2])
    elif len(sys.argv) >= 7 and sys.argv[1] == "pmc":
        pmc(sys.argv[2], sys.argv[3], int(sys.argv[4]), sys.argv[5], sys.argv[6])
    elif len(sys.argv) >= 4 and sys.argv[1] == "instep":
        instep(sys.argv[2], int(sys.argv[3]))
    elif len(sys.argv) >= 5 and sys.argv[1] == "pmctable":
        pmctable(sys.argv[2], sys.argv[3], int(sys.argv[4]), int(sys.argv[5]) if len(sys.argv) > 5 else None)
    elif len(sys.argv) >= 4 and sys.argv[1] == "sq":
        sq(sys.argv[2], sys.argv[3])
    elif len(sys.argv) >= 5 and sys.argv[1] == "mfma":
        mfma(sys.argv[2], sys.argv[3], sys.argv[4])
    else:
        print(__doc__)
        sys.exit(2)
