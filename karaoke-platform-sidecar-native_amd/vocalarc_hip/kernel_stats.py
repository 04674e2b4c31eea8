"""Summarise rocprofv3 runs as markdown.

bench.py under `rocprofv3 --kernel-trace --stats`: reads `*_kernel_stats.csv`
from the run directory and the bench.py JSON line the same command printed,
and writes a short table (kernel, calls, total and average duration, share)
plus the live HIP-event figure of the dominant kernel for comparison:

    python -m vocalarc_hip.kernel_stats RUN_DIR BENCH_JSON OUT.md "<command>"

kernel_bench under `rocprofv3 --kernel-trace`: pairs every kernel_bench
record that names its device kernels with the trace's dispatches of those
kernels, in order (the record's warm-up dispatches first, then its timed
ones), and reports the rocprofv3 average per call beside the live HIP-event
figure, with the achieved rate and fraction of peak from the record's
algorithmic work:

    python -m vocalarc_hip.kernel_stats kernels RUN_DIR BENCH_JSONL OUT.md "<command>"

The reference host linked against the HIP provider under `rocprofv3
--kernel-trace --memory-copy-trace`: splits the trace into the host's
requests at idle gaps of the device (> 20 ms), and reports per request the
kernel and copy time beside the host's own `inferenceMs` from its responses:

    python -m vocalarc_hip.kernel_stats host RUN_DIR RESPONSES_JSONL OUT.md "<commands>"

`rocprofv3 --pmc` passes (one directory each): the per-dispatch average of
every counter over the dispatches whose kernel name matches a regular
expression (optionally only those with a given grid size):

    python -m vocalarc_hip.kernel_stats counters KERNEL_REGEX OUT.md "<commands>" DIR [DIR ...]
"""

from __future__ import annotations

import csv
import json
import re
import sys
from pathlib import Path

# kernel-name patterns (demangled or mangled) -> what the launch computes in
# the separation pass
ROLES = [
    (r"gemm_h2_kernel(<|ILi)4", "FFN up-projection + GELU-GLU (fp32 via two-piece fp16)"),
    (r"gemm_h2_kernel(<3, true|ILi3ELb1E)",
     "out projection + residual, A as the attentions' h2 rows (fp32 via two-piece fp16)"),
    (r"gemm_h2_kernel(<3, false|ILi3ELb0E)",
     "FFN down-projection + residual, raising the stream's bound (fp32 via two-piece fp16)"),
    (r"gemm_h2_kernel(<|ILi)3", "out projection / FFN down-projection + residual (fp32 via two-piece fp16)"),
    (r"gemm_h2_kernel(<0, false, true[,>]|ILi0ELb0ELb1E)",
     "time-axis fused QKV + gate projection with the attention's pre-norm inside, k (rotated) and v written as the "
     "attention's fp16 pieces (fp32 via two-piece fp16)"),
    (r"gemm_h2_kernel(<|ILi)0", "fused QKV + gate projection (fp32 via two-piece fp16)"),
    (r"gemm_h2_batched_kernel(<|ILi)2", "mask estimator layer 1 + tanh, batched over bands (fp32 via two-piece fp16)"),
    (r"gemm_h2_batched_kernel(<|ILi)0", "mask estimator layer 2, batched over bands (fp32 via two-piece fp16)"),
    (r"split_weight_h2_kernel", "weight split into fp16 pieces (model load)"),
    (r"scale_columns_kernel", "RMSNorm gain folded into the QKV weight (model load)"),
    (r"interleave_glu_bias_kernel", "GELU-GLU bias interleave (model load)"),
    (r"absmax_kernel", "maxima: of a weight for its fp16 pieces (model load), of the residual stream (once per pass)"),
    (r"absmax_partial_kernel", "residual stream maximum, partial (once per pass)"),
    (r"operand_bounds_kernel", "operand bounds of the fp16 two-piece GEMMs (model load)"),
    (r"attention_h2_kvp_kernel", "time-axis attention, L = 801, on the fused projection's k/v pieces (fp32 via "
     "two-piece fp16)"),
    (r"attention_h2_kernel", "time-axis attention, L = 801 (fp32 via two-piece fp16)"),
    (r"attention_short_h2_kernel", "band-axis attention, L = 62 (fp32 via two-piece fp16)"),
    (r"band_attention_fused_kernel", "band-axis pre-norm q, k, v and gate projection with the attention, L = 62, "
     "one kernel (fp32 via two-piece fp16)"),
    (r"rmsnorm_h2_kernel", "FFN pre-norm, written as fp16 pieces for the FFN-up GEMM"),
    (r"gemm_split_kernel(<|ILi)4", "FFN up-projection + GELU-GLU (fp32 via split bf16)"),
    (r"gemm_split_kernel(<|ILi)3", "out projection / FFN down-projection + residual (fp32 via split bf16)"),
    (r"gemm_split_kernel(<|ILi)0", "fused QKV + gate projection (fp32 via split bf16)"),
    (r"split_weight_kernel", "weight split into bf16 pieces (model load)"),
    (r"gemm_f32_kernel(<|ILi)4", "FFN up-projection + GELU-GLU (fp32)"),
    (r"gemm_f32_kernel(<|ILi)3", "out projection / FFN down-projection + residual (fp32)"),
    (r"gemm_f32_kernel(<|ILi)0", "fused QKV + gate projection (fp32)"),
    (r"gemm_f32_batched_kernel(<|ILi)2", "mask estimator layer 1 + tanh, batched over bands (fp32)"),
    (r"gemm_f32_batched_kernel(<|ILi)0", "band split (and mask layer 2 off the split path), batched over bands (fp32)"),
    (r"gemm_bf16_(dma_)?kernel(<|ILi)4", "FFN up-projection + GELU-GLU (bf16 variant)"),
    (r"gemm_bf16_(dma_)?kernel(<|ILi)3", "out / FFN down-projection + residual (bf16 variant)"),
    (r"gemm_bf16_(dma_)?kernel(<|ILi)0", "fused QKV + gate projection (bf16 variant)"),
    (r"gemm_bf16_(dma_)?batched_kernel(<|ILi)2", "mask layer 1 (bf16 variant)"),
    (r"gemm_bf16_(dma_)?batched_kernel(<|ILi)0", "band split / mask layer 2 (bf16 variant)"),
    (r"attention_bf16_kernel(<|ILi)4", "time-axis attention, L = 801 (bf16 variant)"),
    (r"attention_bf16_kernel(<|ILi)2", "band-axis attention, L = 62 (bf16 variant)"),
    (r"attention_split_kernel", "time-axis attention, L = 801 (fp32 via split bf16)"),
    (r"attention_kernel(<|ILi)4", "time-axis attention, L = 801"),
    (r"attention_short_kernel", "band-axis attention, L = 62"),
    (r"rmsnorm_kernel", "pre-norms and final norm"),
    (r"istft_frames_kernel", "mask multiply + inverse FFT"),
    (r"stft_kernel", "STFT"),
    (r"ola_kernel", "overlap-add"),
    (r"band_gather_norm_kernel", "band gather + RMSNorm"),
    (r"mask_glu_scatter_kernel", "mask GLU + bin scatter"),
    (r"crossfade_kernel", "window cross-fade"),
    (r"to_bf16_kernel", "bf16 weight copies (once per model)"),
    (r"unpack_weight_kernel", "weight upload (once per model)"),
]


def role(name: str) -> str:
    for pat, what in ROLES:
        if re.search(pat, name):
            return what
    return ""


def kernels(run_dir: str, jsonl: str, out: str, command: str) -> int:
    path = next(Path(run_dir).rglob("*kernel_trace.csv"))
    trace = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    recs = [json.loads(x) for x in Path(jsonl).read_text().splitlines() if x.startswith("{")]
    lines = [
        "# Per-kernel rocprofv3 time against the roofline (kernel_bench, command below)", "",
        "Commands (repository root, MI355X box):", "", "```", command.strip(), "```", "",
        f"Source: `{path.name}` (rocprofv3 kernel trace) paired in order with the kernel_bench JSON lines of the "
        "same run: each record's device kernels, its warm-up dispatches, then its timed ones. `rocprof ms` is the "
        "average per call over the timed dispatches (sum of the kernels one call launches); `live ms` is the "
        "HIP-event mean over the same calls. Rates use the algorithmic work (each tensor read and written once; "
        "2*M*K*N per GEMM); `frac` is against 8 TB/s HBM or the matrix-core peak of the instruction the kernel "
        "runs (fp32 MFMA 157.3 TFLOP/s; bf16/fp16 2.5 PFLOP/s, times the piece products per fp32 product).", "",
        "| kernel | shape | rocprof ms | live ms | algorithmic work | achieved | frac of peak |",
        "|---|---|---:|---:|---:|---:|---:|",
    ]
    pos = 0
    for r in recs:
        rx = r.get("device")
        live = r["ms"]
        prof = None
        if rx:
            pat = re.compile(rx)
            got = []
            i = pos
            while i < len(trace) and len(got) < r["dispatches"]:
                if pat.search(trace[i]["Kernel_Name"]):
                    got.append(trace[i])
                i += 1
            if len(got) == r["dispatches"]:
                pos = i
                timed = got[-r["timed_dispatches"]:]
                ns = sum(int(t["End_Timestamp"]) - int(t["Start_Timestamp"]) for t in timed)
                prof = ns / 1e6 / _timed_calls(r)
        ms = prof if prof is not None else live
        if "algorithmic_GB" in r and r.get("bound") == "hbm":
            rate = r["algorithmic_GB"] / (ms * 1e-3)
            work, ach, frac = f"{r['algorithmic_GB']:.3f} GB", f"{rate:.0f} GB/s", rate / 8000.0
        elif "algorithmic_GFLOP" in r:
            tf = r["algorithmic_GFLOP"] / (ms * 1e-3) / 1e3
            k = r.get("mc_products", 1)
            work = f"{r['algorithmic_GFLOP']:.1f} GFLOP"
            ach = f"{tf:.1f} TFLOP/s" + (f" (x{k} = {k * tf:.0f} on the matrix cores)" if k > 1 else "")
            frac = k * tf / r.get("peak_TFLOP_per_s", 157.3)
        else:
            work, ach, frac = "", "", None
        lines.append(f"| {r['kernel']} | {r['shape']} | {'' if prof is None else f'{prof:.4f}'} | {live:.4f} | "
                     f"{work} | {ach} | {'' if frac is None else f'{frac:.3f}'} |")
    Path(out).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


XCDS = 8              # GRBM_GUI_ACTIVE is summed over the XCDs
SIMDS_PER_SE = 32     # SQ_CYCLES is summed over the 32 shader engines, 32 SIMDs each
PEAK_CLOCK_GHZ = 2.4  # the clock of the published dense MFMA peaks


def counters(regex: str, out: str, command: str, *dirs: str) -> int:
    """Summary of a kernel's counters over the dispatches whose name matches
    regex; with a regex ending in "#largest", only the dispatches of the
    largest grid (the full 8-window passes of a separation run)."""
    largest = regex.endswith("#largest")
    regex = regex[:-len("#largest")] if largest else regex
    pat = re.compile(regex)
    vals: dict[str, list[float]] = {}
    names = set()
    per_dispatch: dict[tuple[int, str], dict[str, float]] = {}
    rows_all = []
    for i, d in enumerate(dirs):
        path = next(Path(d).rglob("*counter_collection.csv"))
        rows_all += [(i, r) for r in csv.DictReader(open(path)) if pat.search(r["Kernel_Name"])]
    grid_max = max((int(r["Grid_Size"]) for _, r in rows_all), default=0)
    for i, r in rows_all:
        if largest and int(r["Grid_Size"]) != grid_max:
            continue
        if True:
            names.add(r["Kernel_Name"])
            vals.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
            rec = per_dispatch.setdefault((i, r["Dispatch_Id"]), {})
            rec["ns"] = float(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
            rec[r["Counter_Name"]] = float(r["Counter_Value"])
    avg = {k: sum(v) / len(v) for k, v in vals.items()}
    lines = [f"# rocprofv3 counters of `{regex}`", "", "Commands (repository root, MI355X box; one pass per counter "
             "group):", "", "```", command.strip(), "```", "",
             "Kernels matched: " + ", ".join(f"`{n[:120]}`" for n in sorted(names)) +
             (f" (only the dispatches of the largest grid, {grid_max} work-items)" if largest else ""), "",
             "Per-dispatch averages (totals over the device as rocprofv3 reports them):", "",
             "| counter | value |", "|---|---:|"]
    for k in sorted(avg):
        lines.append(f"| `{k}` | {avg[k]:.4g} |")
    # dispatches of the pass that read the clock and the matrix-core busy
    # cycles: the clock each ran at (GRBM_GUI_ACTIVE per XCD over its
    # duration), the matrix cores' busy share of the SIMD cycles, and their
    # product with clock / peak clock -- the fraction of the dense MFMA peak
    keys = ("GRBM_GUI_ACTIVE", "SQ_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES")
    rows = [(k, v) for k, v in sorted(per_dispatch.items(), key=lambda kv: (kv[0][0], int(kv[0][1])))
            if all(c in v for c in keys) and v["ns"] > 0]
    if rows:
        shown = rows[-12:]
        busy_all = [v["SQ_VALU_MFMA_BUSY_CYCLES"] / (v["SQ_CYCLES"] * SIMDS_PER_SE) for _, v in rows]
        clk_all = sorted(v["GRBM_GUI_ACTIVE"] / XCDS / v["ns"] for _, v in rows)
        lines += ["", f"Over the {len(rows)} dispatches of that pass: matrix cores busy {min(busy_all):.3f}-"
                  f"{max(busy_all):.3f} (mean {sum(busy_all) / len(busy_all):.3f}), clock median "
                  f"{clk_all[len(clk_all) // 2]:.3f} GHz" + (f"; the last {len(shown)} below" if len(shown) < len(rows)
                                                             else "") + "."]
        rows = shown
        lines += ["", "Per dispatch (the pass with the clock and busy counters): clock = `GRBM_GUI_ACTIVE` / "
                  f"{XCDS} XCDs / duration; busy = `SQ_VALU_MFMA_BUSY_CYCLES` / (`SQ_CYCLES` x {SIMDS_PER_SE}); "
                  f"fraction of the MFMA peak = busy x clock / {PEAK_CLOCK_GHZ} GHz. Durations are the profiled "
                  "dispatches' own (serialised, with pauses between them, so the clock ramps up over the first "
                  "ones).", "",
                  "| dispatch | ms | cycles per XCD | clock GHz | matrix cores busy | fraction of peak |",
                  "|---:|---:|---:|---:|---:|---:|"]
        for (_, did), v in rows:
            cyc = v["GRBM_GUI_ACTIVE"] / XCDS
            clk = cyc / v["ns"]
            busy = v["SQ_VALU_MFMA_BUSY_CYCLES"] / (v["SQ_CYCLES"] * SIMDS_PER_SE)
            lines.append(f"| {did} | {v['ns'] / 1e6:.3f} | {cyc:.4g} | {clk:.3f} | {busy:.3f} | "
                         f"{busy * clk / PEAK_CLOCK_GHZ:.3f} |")
    Path(out).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


def host(run_dir: str, responses: str, out: str, command: str) -> int:
    ktrace = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"])
              for r in csv.DictReader(open(next(Path(run_dir).rglob("*kernel_trace.csv"))))]
    ctrace = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r.get("Direction", r.get("Operation", "")))
              for r in csv.DictReader(open(next(Path(run_dir).rglob("*memory_copy_trace.csv"))))]
    events = sorted([(a, b, "k", n) for a, b, n in ktrace] + [(a, b, "c", n) for a, b, n in ctrace])
    groups, cur, last = [], [], None
    for e in events:
        if last is not None and e[0] - last > 20_000_000:
            groups.append(cur)
            cur = []
        cur.append(e)
        last = e[1] if last is None else max(last, e[1])
    if cur:
        groups.append(cur)
    sep = [json.loads(x) for x in Path(responses).read_text().splitlines() if x.strip()]
    sep = [r for r in sep if r.get("type") == "separated"]
    lines = ["# The reference host with the HIP provider: device time per request (command below)", "",
             "Commands (repository root, MI355X box):", "", "```", command.strip(), "```", "",
             "Source: the rocprofv3 kernel and memory-copy traces, split into requests at idle gaps of the device "
             "(> 20 ms); `inferenceMs` is the host's own timing of the request (STFT to iSTFT, "
             "native/vocalarc_separation.c:1584-1586) from its responses, in order. The first request also uploads, "
             "splits and bounds the weights (first use of the cached tensors).", "",
             "| request | inferenceMs | device span ms | kernels ms | copies ms (count) | kernel classes (ms) |",
             "|---:|---:|---:|---:|---:|---|"]
    for i, g in enumerate(groups):
        kern = sum(b - a for a, b, t, _ in g if t == "k") / 1e6
        cop = [b - a for a, b, t, _ in g if t == "c"]
        span = (max(b for _, b, _, _ in g) - min(a for a, _, _, _ in g)) / 1e6
        by: dict[str, float] = {}
        for a, b, t, n in g:
            if t == "k":
                key = re.sub(r"\(.*", "", n).replace("void ", "")
                by[key] = by.get(key, 0.0) + (b - a) / 1e6
        top = "; ".join(f"{k} {v:.1f}" for k, v in sorted(by.items(), key=lambda kv: -kv[1])[:5])
        inf = f"{float(sep[i]['inferenceMs']):.1f}" if i < len(sep) and "inferenceMs" in sep[i] else ""
        lines.append(f"| {i + 1} | {inf} | {span:.1f} | {kern:.1f} | {sum(cop) / 1e6:.1f} ({len(cop)}) | {top} |")
    Path(out).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


def _timed_calls(r: dict) -> int:
    """Timed calls of a record: its timed dispatches over the dispatches one
    call launches (dispatches = calls made x per call)."""
    per_call = r.get("per_call", 1)
    return max(1, r["timed_dispatches"] // per_call)


def main() -> int:
    if sys.argv[1] == "kernels":
        return kernels(*sys.argv[2:6])
    if sys.argv[1] == "host":
        return host(*sys.argv[2:6])
    if sys.argv[1] == "counters":
        return counters(sys.argv[2], sys.argv[3], sys.argv[4], *sys.argv[5:])
    run_dir, bench_json, out, command = sys.argv[1:5]
    path = next(Path(run_dir).rglob("*kernel_stats.csv"))
    rows = list(csv.DictReader(open(path)))
    bench = None
    for line in Path(bench_json).read_text().splitlines():
        if line.startswith("{"):
            bench = json.loads(line)
    lines = [
        "# Kernel time of the 5-minute separation (bench.py, command below)",
        "", "Command (repository root, MI355X box):", "", "```", command.strip(), "```", "",
        f"Source: `{path.name}` written by rocprofv3 (durations in ms). The run covers model load, the warm-up and "
        "the timed steps of bench.py (and those of the precision variants when the command runs them).", "",
        "| kernel | role | calls | total ms | avg ms | % |", "|---|---|---:|---:|---:|---:|",
    ]
    for r in rows:
        name = r["Name"]
        short = name if len(name) < 90 else name[:87] + "..."
        lines.append(f"| `{short}` | {role(name)} | {r['Calls']} | {float(r['TotalDurationNs']) / 1e6:.2f} | "
                     f"{float(r['AverageNs']) / 1e6:.4f} | {float(r['Percentage']):.2f} |")
    if bench:
        rf = bench["roofline"]
        dom = next((r for r in rows if re.search(ROLES[0][0], r["Name"])), None)
        lines += ["", f"Dominant kernel: live HIP-event average in bench.py {rf['avg_launch_ms']} ms over "
                      f"{rf['launches']} launches of the timed region; rocprofv3 average over all its launches "
                      f"{float(dom['AverageNs']) / 1e6:.4f} ms ({dom['Calls']} launches)." if dom else "",
                  "", "bench.py line of the same command:", "", "```", json.dumps(bench), "```"]
    Path(out).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


if __name__ == "__main__":
    sys.exit(main())
