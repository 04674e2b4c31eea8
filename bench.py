#!/usr/bin/env python3
"""Benchmark: realtime factor of the full separation path on one MI355X.

Workload (one "step"): separate a 5-minute stereo 44.1 kHz seeded mix (6 sine
partials per channel + white noise) with a random-init BS-RoFormer of dim 384,
depth 12, 62 bands, 8 heads x 64, GELU-GLU FFN (mult 4), hop 441, n_fft 2048:
8 s windows with 2 s overlap (50 windows), 8 windows per device pass, linear
cross-fade.  The input waveform is resident in HBM when the timed region
starts; the output waveform is in HBM when it ends.  fp32 accuracy for
`value`: the transformer and mask-estimator linears and the attention
products of both axes run on the fp16 matrix cores as two-piece splits of
their power-of-two-scaled fp32 operands (three piece products per fp32
product, fp32 accumulation), everything else on fp32 MFMA / fp32 / fp64.
Timed after it and reported separately: "fp32_mfma_variant", the same job
with every product on the fp32 MFMA instruction, and "bf16_variant" (bf16
operands at the matrix cores, fp32 accumulation and everything else fp32),
each with its difference from the `value` output.

value = audio seconds separated per wall second (realtime factor).
roofline: the dominant kernel (the FFN up-projection GEMM with the GELU-GLU
epilogue), timed with HIP events on the launch stream inside the timed
region.  Its algorithm computes every fp32 product as three fp16 piece
products, so its matrix-core work is 3 * 2*M*K*N FLOP per launch, priced
against the 2.5 PFLOP/s dense fp16 MFMA peak; the fp32-equivalent rate
(2*M*K*N per launch) is reported beside it.
cpu_baseline: the oracle (C restatement of the reference CPU path) on the
host cores: one whole 8 s window at depth 12, timed, times the job's window
count (windows are independent).
host_path: the reference C11 host on a 10 s input at the reference model
shape, as the reference CPU executable and linked against the HIP provider
(one warm-up request, median inferenceMs of three:
native/scripts/benchmark.py:135-161), with the CPU model and core counts.

    python bench.py [--gpus 1] [--steps 3] [--warmup 1]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "karaoke-platform-sidecar-native_amd"))

SECONDS = 300.0
CHUNK_S, STEP_S, BATCH = 8.0, 6.0, 8
RATE = 44_100
MFMA_FP32_PEAK_TFLOPS = 157.3
MFMA_BF16_PEAK_TFLOPS = 2500.0
MFMA_FP16_PEAK_TFLOPS = 2500.0
H2_PRODUCTS = 3  # fp16 piece products per fp32 product in the two-piece GEMM
HBM_PEAK_GBS = 8000.0
HOST_SECONDS = 10.0
DOMINANT = "gemm_ff1"
KERNEL_CLASSES = ("stft", "band_gather", "gemm_band_split", "rmsnorm", "gemm_qkv", "attention_long",
                  "attention_short", "band_attention", "gemm_out", "gemm_ff1", "gemm_ff2", "gemm_mask1", "gemm_mask2", "mask_glu",
                  "istft", "crossfade")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def ff1_flops_per_step(d, chunk: int, step: int, length: int, batch: int) -> float:
    count = 1 if length <= chunk else 1 + (length - chunk + step - 1) // step
    T = d.frames(chunk)
    flops = 0.0
    for k0 in range(0, count, batch):
        n = min(batch, count - k0)
        M = n * T * d.bands
        flops += 2 * d.depth * (2.0 * M * d.dim * d.ff1_out)  # time + band axis per layer
    return flops


def cpu_baseline(d, blob, x, chunk: int, step: int, threads: int) -> dict:
    """Oracle (OpenMP) on one whole 8 s window of the job at full depth: STFT,
    band split, every axial layer, mask estimator and iSTFT, timed; the job is
    that times its window count (the windows are independent)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import numpy as np
    import oracle as O

    O.set_threads(threads)
    m = O.Model(d, blob)
    w = np.ascontiguousarray(x[:, :chunk])
    t0 = time.perf_counter()
    m.forward(w)
    per_window = time.perf_counter() - t0
    count = 1 + (x.shape[1] - chunk + step - 1) // step
    job = per_window * count
    return {
        "value": round(x.shape[1] / RATE / job, 4),
        "unit": "audio s / wall s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle (C restatement of the reference CPU path, OpenMP, {threads} threads) on one whole "
                   f"{chunk / RATE:.0f} s window at depth {d.depth}: {per_window:.2f} s; times {count} windows "
                   f"= {job:.0f} s for the {x.shape[1] / RATE:.0f} s job"),
    }


def cpu_info() -> dict:
    """CPU model and core counts of this host (the thread counts the host
    path uses): logical = CPUs this process may run on (nproc), physical =
    distinct (package, core) pairs among them."""
    logical = sorted(os.sched_getaffinity(0))
    model, cores = None, set()
    try:
        blocks = Path("/proc/cpuinfo").read_text().split("\n\n")
    except OSError:
        blocks = []
    for blk in blocks:
        kv = {}
        for line in blk.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                kv[k.strip()] = v.strip()
        if "processor" not in kv:
            continue
        model = model or kv.get("model name")
        if int(kv["processor"]) in logical:
            cores.add((kv.get("physical id", "0"), kv.get("core id", kv["processor"])))
    return {"model": model, "logical_cpus": len(logical), "physical_cores": len(cores) or len(logical),
            "os_cpu_count": os.cpu_count()}


def host_path(seconds: float) -> dict:
    """The reference C11 host, unchanged, on a config-0-recipe input (6 sines
    per channel + N(0, 0.01^2)) with a seeded pack in the reference layout
    (dim 256, depth 16, 90 bands, hop 512): the reference CPU executable at
    the logical and the physical core count, and the same host linked
    against the HIP provider; each one warm-up request, then the median
    inferenceMs (forward_model: STFT to iSTFT, native/vocalarc_separation.c:
    1584-1586) of three (native/scripts/benchmark.py:135-161).  The runtime
    label follows benchmark.py:171 with the HIP backend counted as a GPU
    runtime."""
    import shutil
    import tempfile

    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O
    from vocalarc_hip import audio, pack
    from vocalarc_hip.dims import REFERENCE_DIMS

    for exe in (O.REF_EXE, O.REF_GPU_EXE):
        if not exe.exists():
            return {"skipped": f"{exe.relative_to(ROOT)} not built (make -C oracle ref gpu-host)"}
    info = cpu_info()
    tmp = Path(tempfile.mkdtemp(prefix="vocalarc-bench-host-"))
    try:
        pack_path = tmp / "model.f32"
        pack.write_pack(pack_path, pack.synthetic_pack(REFERENCE_DIMS, 1234))
        wav = tmp / "in.wav"
        x = audio.sine_mix(seconds, 2026)
        audio.write_wav_float(wav, x)

        def run(exe, threads, tag):
            v, i = tmp / f"{tag}-v.wav", tmp / f"{tag}-i.wav"
            t0 = time.perf_counter()
            resp = O.run_reference(exe, pack_path, wav, v, i, threads=threads, repetitions=4, timeout=1800)
            wall = time.perf_counter() - t0
            sep = [r for r in resp if r.get("type") == "separated"]
            if len(sep) != 4 or not all(r.get("ok") for r in sep):
                raise RuntimeError(f"{tag}: {resp}")
            ms = [float(r["inferenceMs"]) for r in sep[1:]]
            med = float(np.median(ms))
            backend = sep[-1].get("backend", "")
            log(f"host path {tag}: {threads} threads, inferenceMs {ms} ({wall:.1f} s wall)")
            return {"backend": backend, "device": sep[-1].get("device"),
                    "runtime": "vocalarc-native-gpu" if backend != "native-cpu" else "vocalarc-native-cpu",
                    "threads": threads, "inference_ms": [round(t, 2) for t in ms], "median_ms": round(med, 2),
                    "rtf": round(seconds / (med * 1e-3), 3)}, audio.read_wav_float(v)[0], \
                audio.read_wav_float(i)[0]

        gpu, gv, gi = run(O.REF_GPU_EXE, info["logical_cpus"], "hip")
        cpu_runs = []
        cv = ci = None
        for threads in sorted({info["logical_cpus"], info["physical_cores"]}, reverse=True):
            r, v, i = run(O.REF_EXE, threads, f"cpu{threads}")
            cpu_runs.append(r)
            if cv is None:
                cv, ci = v, i
        parity = {}
        for name, ref, out in (("vocals", cv, gv), ("instrumental", ci, gi)):
            cmp = audio.compare(ref, out)
            parity[name] = {"max_abs": cmp["max_abs"], "snr_db": round(cmp["snr_db"], 2)}
        return {
            "workload": f"reference host, {seconds:.0f} s stereo 44.1 kHz, seeded pack at the reference shape "
                        f"(dim 256, depth 16, 90 bands, hop 512, T = {REFERENCE_DIMS.frames(x.shape[1])})",
            "cpu": info,
            "hip_provider": gpu,
            "reference_cpu": cpu_runs,
            "speedup_vs_cpu": round(cpu_runs[0]["median_ms"] / gpu["median_ms"], 2),
            "parity_vs_reference_cpu": parity,
        }
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def measured_traffic() -> tuple[int | None, str | None]:
    """HBM bytes per launch of the dominant kernel, from the committed
    calibrated rocprofv3 counter summary (FETCH_SIZE/WRITE_SIZE scaled by a
    plain copy); None if that summary is absent."""
    path = ROOT / "profiles" / "gemm-h2-ff1-geglu_traffic.md"
    if not path.exists():
        return None, None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1]), str(path.relative_to(ROOT))
    return None, None


def variant(ctx, model, dx, dv, ref_out, length, chunk, step, args, d, precision, label) -> dict:
    """The same job in another precision mode; its difference from the default output."""
    import numpy as np
    import torch

    from vocalarc_hip import native

    model.set_precision(precision)
    steps, warmup = min(args.steps, 5), min(args.warmup, 1)
    for i in range(warmup):
        model.separate(dx, length, chunk, step, BATCH, dv)
        ctx.sync()
    if args.breakdown:
        log(f"{label} step by kernel class: " + breakdown(ctx, lambda: model.separate(dx, length, chunk, step, BATCH, dv)))
    ctx.timing(DOMINANT)
    ctx.timing_reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        model.separate(dx, length, chunk, step, BATCH, dv)
    ctx.sync()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ctx.timing(None)
    ms, launches = ctx.timing_get(DOMINANT)
    model.set_precision(native.PRECISION_FP32)
    log(f"{label}: timed {steps} steps: {wall:.3f} s")
    out = dv.cpu().numpy().astype(np.float64)
    ref = ref_out.astype(np.float64)
    snr = 10 * np.log10(np.sum(ref * ref) / max(np.sum((out - ref) ** 2), 1e-300))
    tf = ff1_flops_per_step(d, chunk, step, length, BATCH) * steps / (ms * 1e-3) / 1e12 if ms > 0 else 0.0
    return {
        "value": round(length / RATE * steps / wall, 3),
        "unit": "audio s / wall s",
        "steps": steps,
        "ms_per_step": round(wall / steps * 1e3, 2),
        "snr_db_vs_value_output": round(float(snr), 2),
        "max_abs_vs_value_output": float(np.max(np.abs(out - ref))),
        "dominant_kernel_tflops": round(tf, 2),
        "dominant_avg_launch_ms": round(ms / max(launches, 1), 4),
    }


def bf16_variant(ctx, model, dx, dv, ref_out, length, chunk, step, args, d) -> dict:
    """The same job with bf16 matrix-core operands; SNR against the fp32 output."""
    from vocalarc_hip import native

    v = variant(ctx, model, dx, dv, ref_out, length, chunk, step, args, d, native.PRECISION_BF16, "bf16 variant")
    tf = v.pop("dominant_kernel_tflops")
    return {
        "value": v["value"], "unit": v["unit"], "steps": v["steps"], "ms_per_step": v["ms_per_step"],
        "dtype": "bf16 MFMA operands, fp32 accumulation",
        "snr_db_vs_fp32": v["snr_db_vs_value_output"],
        "dominant_kernel": {"kernel": "gemm_bf16_dma_kernel<GELU-GLU>", "achieved": tf,
                            "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                            "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                            "avg_launch_ms": v["dominant_avg_launch_ms"]},
    }


def fp32_mfma_variant(ctx, model, dx, dv, ref_out, length, chunk, step, args, d) -> dict:
    """The same job with every product on the fp32 MFMA instruction."""
    from vocalarc_hip import native

    v = variant(ctx, model, dx, dv, ref_out, length, chunk, step, args, d, native.PRECISION_FP32_MFMA,
                "fp32 MFMA variant")
    tf = v.pop("dominant_kernel_tflops")
    v["dtype"] = "fp32 (v_mfma_f32_32x32x2f32 for every product)"
    v["dominant_kernel"] = {"kernel": "gemm_f32_kernel<GELU-GLU>", "achieved": tf, "peak": MFMA_FP32_PEAK_TFLOPS,
                            "unit": "TFLOP/s", "frac": round(tf / MFMA_FP32_PEAK_TFLOPS, 4),
                            "avg_launch_ms": v.pop("dominant_avg_launch_ms")}
    return v


def breakdown(ctx, run) -> str:
    """Per-kernel-class device time of one step (HIP events around each launch)."""
    ctx.timing("*")
    ctx.timing_reset()
    run()
    ctx.sync()
    ctx.timing(None)
    rows = [(name, *ctx.timing_get(name)) for name in KERNEL_CLASSES]
    total = sum(ms for _, ms, _ in rows) or 1.0
    return "; ".join(f"{name} {ms:.1f} ms ({100 * ms / total:.1f}%)" for name, ms, n in rows if n)


def _final_gamma(d, blob):
    from vocalarc_hip import pack
    return pack.tensor_views(d, blob)["final_gamma"]


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--seconds", type=float, default=SECONDS)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-host-path", action="store_true", help="skip the reference-host (config 0) leg")
    ap.add_argument("--host-seconds", type=float, default=HOST_SECONDS)
    ap.add_argument("--no-bf16", action="store_true", help="skip the bf16-MFMA variant")
    ap.add_argument("--no-variants", action="store_true", help="skip the fp32-MFMA and bf16 variants")
    ap.add_argument("--breakdown", action="store_true", help="per-kernel-class time of one untimed step (stderr)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build runs the separation path on a single GPU "
              "(sharding the windows over several GPUs is not implemented)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from vocalarc_hip import audio, native, pack
    from vocalarc_hip.dims import CONFIG_DIMS

    host = None
    if not args.no_host_path:
        # before this process touches the GPU: the executables run as children
        log(f"host path: reference host on {args.host_seconds:.0f} s (CPU executable and HIP provider) ...")
        try:
            host = host_path(args.host_seconds)
        except Exception as e:  # noqa: BLE001  (reported in the line, the GPU bench goes on)
            host = {"error": f"{type(e).__name__}: {e}"[:500]}

    d = CONFIG_DIMS
    chunk, step = int(CHUNK_S * RATE), int(STEP_S * RATE)
    log("generating synthetic pack and input ...")
    blob = pack.synthetic_pack(d, 2026)
    x = audio.sine_mix(args.seconds, 300)
    length = x.shape[1]

    ctx = native.Context()
    model = native.Model(ctx, d, blob)
    dx = torch.from_numpy(x).to("cuda:0")
    dv = torch.empty_like(dx)
    torch.cuda.synchronize()

    for i in range(args.warmup):
        t0 = time.perf_counter()
        model.separate(dx, length, chunk, step, BATCH, dv)
        ctx.sync()
        log(f"warmup step {i}: {time.perf_counter() - t0:.3f} s")
    if args.breakdown:
        log("fp32 step by kernel class: " + breakdown(ctx, lambda: model.separate(dx, length, chunk, step, BATCH, dv)))

    ctx.timing(DOMINANT)
    ctx.timing_reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        model.separate(dx, length, chunk, step, BATCH, dv)
    ctx.sync()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ctx.timing(None)
    ms, launches = ctx.timing_get(DOMINANT)
    log(f"timed {args.steps} steps: {wall:.3f} s")

    out = dv.cpu().numpy()
    assert np.all(np.isfinite(out)), "non-finite output"

    flops = ff1_flops_per_step(d, chunk, step, length, BATCH) * args.steps
    achieved = flops / (ms * 1e-3) / 1e12 if ms > 0 else 0.0
    traffic, traffic_src = measured_traffic()
    alg_bytes = 3.058e9  # A 610 MB + weight pieces 4.7 MB + output 2.44 GB per full 8-window launch
    mc = H2_PRODUCTS * achieved  # matrix-core FLOP/s the algorithm executes
    roofline = {
        "kernel": "gemm_h2_kernel<GELU-GLU> (FFN up-projection, M=397296 K=384 N=3072 per 8-window pass)",
        "bound": "mfma",
        "achieved": round(mc, 2),
        "peak": MFMA_FP16_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(mc / MFMA_FP16_PEAK_TFLOPS, 4),
        "note": "fp32 products computed as 3 fp16 piece products each (two-piece splits of power-of-two-scaled "
                "operands, v_mfma_f32_32x32x16_f16, fp32 accumulation): achieved = 3 x 2*M*K*N FLOP per launch "
                "over the launch time, against the dense fp16 MFMA peak",
        "fp32_equivalent_tflops": round(achieved, 2),
        "fp32_equivalent_ceiling_tflops": round(MFMA_FP16_PEAK_TFLOPS / H2_PRODUCTS, 1),
        "traffic": traffic,
        "traffic_unit": "bytes per full 8-window launch (FETCH_SIZE + WRITE_SIZE, calibrated by a device copy)",
        "traffic_algorithmic": alg_bytes,
        "traffic_ratio": round(traffic / alg_bytes, 3) if traffic else None,
        "traffic_source": traffic_src,
        "launches": launches,
        "avg_launch_ms": round(ms / max(launches, 1), 4),
    }

    fp32_mfma = None
    if not args.no_variants:
        fp32_mfma = fp32_mfma_variant(ctx, model, dx, dv, out, length, chunk, step, args, d)
    bf16 = None
    if not args.no_variants and not args.no_bf16:
        bf16 = bf16_variant(ctx, model, dx, dv, out, length, chunk, step, args, d)

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle) ...")
        cpu = cpu_baseline(d, blob, x, chunk, step, min(16, len(os.sched_getaffinity(0))))

    audio_s = length / RATE * args.steps
    line = {
        "metric": "realtime factor (audio s / wall s) on 1xMI355X; kernel HBM GB/s & MFMA % of peak",
        "value": round(audio_s / wall, 3),
        "unit": "audio s / wall s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "precision_note": "fp32 accuracy: transformer and mask-estimator linears as 2-piece fp16 splits of "
                          "power-of-two-scaled operands (3 products, fp32 accumulation; error vs fp64 at or below "
                          "the fp32 MFMA GEMM's), time- and band-axis attention the same way (bound from the "
                          "QKV projection's weights), band split on fp32 MFMA, DSP in fp64/fp32",
        "data": "synthetic (seeded sine+noise mix, random-init weights N(0,0.02), gammas N(1,0.02))",
        "config": {
            "workload": "full BS-RoFormer separation, 5 min stereo 44.1 kHz, 8 s windows / 2 s overlap, "
                        "8 windows per device pass",
            "audio_seconds": round(length / RATE, 3),
            "dim": d.dim, "depth": d.depth, "bands": d.bands, "heads": d.heads, "dim_head": d.dim_head,
            "ffn": "GELU-GLU x4", "n_fft": d.n_fft, "hop": d.hop, "windows_per_pass": BATCH,
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "host_path": host,
        "fp32_mfma_variant": fp32_mfma,
        "bf16_variant": bf16,
    }
    print(json.dumps(line), flush=True)
    model.close()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
