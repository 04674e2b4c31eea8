"""Per-kernel throughput on one MI355X against the roofline.

Isolated kernels (fp32, inputs N(0,1), gammas N(1,0.02)):
  RMSNorm [49662, 384]; row softmax [496, 801, 801]; rotary [62,8,801,64] and
  [801,8,62,64]; GELU-GLU [49662, 3072] -> [49662, 1536]; residual add
  [49662, 384].
One axial layer at dim 384 (weights N(0,0.02), activations N(0,1)):
  time transformer (62 sequences x 801), band transformer (801 x 62).
Front/back end on 60 s of audio (hop 441, n_fft 2048, 62 bands), spectra in
the pipeline's frame-major layout: STFT, complex mask multiply + iSTFT +
overlap-add, band split, mask estimator.

Work per launch is algorithmic (each tensor read and written once; 2*M*K*N
per GEMM); time is the mean over repetitions measured with HIP events on the
launch stream.  The isolated elementwise kernels cycle over at least four
buffer sets of at least 1 GB together, so no repetition finds its operands
in the 256 MB Infinity Cache (cold-cache HBM figures).  One JSON line per
kernel on stdout; each names the device kernel it times ("device", a regular
expression) and how many of its dispatches the record made ("dispatches":
warm-up, then the timed ones), so kernel_stats can pair it with a
rocprofv3 kernel trace of the same run.

    PYTHONPATH=karaoke-platform-sidecar-native_amd python -m vocalarc_hip.kernel_bench
"""

from __future__ import annotations

import argparse
import json
import sys

import numpy as np

HBM_GBS = 8000.0
FP32_TFLOPS = 157.3
BF16_TFLOPS = 2500.0
FP16_TFLOPS = 2500.0


def _event_time(fn, reps: int) -> tuple[float, int]:
    """(mean ms per call, calls made) of `fn` after untimed calls (see _event_time_sets)."""
    return _event_time_sets([fn], reps)


WARM_MS = 25.0  # untimed work before each record's timed calls


def _event_time_sets(fns, reps: int) -> tuple[float, int]:
    """Mean ms per call over `reps` calls cycling through `fns` (one per
    buffer set), after untimed rounds over all of them: one (which also
    builds per-length tables), then as many as fill WARM_MS -- the clock dips
    for some 10-20 ms when matrix work resumes after a pause (host-side
    set-up), and a record of 5 timed 1.5 ms calls would measure the dip.
    Returns (ms, calls made)."""
    import torch
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for fn in fns:
        fn()
    b.record()
    b.synchronize()
    rounds = 1 + min(200, int(WARM_MS / max(a.elapsed_time(b), 1e-3)))
    for _ in range(rounds - 1):
        for fn in fns:
            fn()
    torch.cuda.synchronize()
    a.record()
    for i in range(reps):
        fns[i % len(fns)]()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) / reps, rounds * len(fns) + reps


def _sets_for(footprint_bytes: float) -> int:
    """Buffer sets for a cold-cache measurement: at least 4, and at least
    1 GB in all (four times the Infinity Cache)."""
    return max(4, -(-int(1 << 30) // max(1, int(footprint_bytes))))


def _emit(name: str, ms, *, gbytes: float | None = None, gflop: float | None = None, shape: str = "",
          peak_tflops: float = FP32_TFLOPS, extra: dict | None = None, device: str | None = None,
          per_call: int = 1, reps: int | None = None, mc_products: int = 1) -> dict:
    """ms: (mean ms per call, calls made) from _event_time(_sets).  device:
    regular expression of the kernel(s) one call launches, per_call of them
    per call; reps: the timed calls among those made.  mc_products:
    matrix-core products per algorithmic product (3 for the fp16 two-piece
    kernels), giving the matrix-core fraction of peak."""
    ms, calls = ms
    rec = {"kernel": name, "shape": shape, "ms": round(ms, 4)}
    if device:
        rec.update({"device": device, "per_call": per_call, "dispatches": calls * per_call,
                    "timed_dispatches": reps * per_call})
    if gbytes is not None:
        gbs = gbytes / (ms * 1e-3)
        rec.update({"algorithmic_GB": round(gbytes, 4), "GB_per_s": round(gbs, 1),
                    "bound": "hbm", "frac_of_peak": round(gbs / HBM_GBS, 4)})
    if gflop is not None:
        tf = gflop / (ms * 1e-3) / 1e3
        rec.update({"algorithmic_GFLOP": round(gflop, 2), "TFLOP_per_s": round(tf, 2), "bound": "mfma",
                    "peak_TFLOP_per_s": peak_tflops, "mc_products": mc_products,
                    "frac_of_peak": round(mc_products * tf / peak_tflops, 4)})
    if extra:
        rec.update(extra)
    print(json.dumps(rec), flush=True)
    return rec


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--only", default="",
                    help="comma list of groups: copy,c1,c2,c3,gemm,ff1,h2,split,attn,bf16,vendor")
    args = ap.parse_args()
    groups = (set(args.only.split(",")) if args.only else
              {"copy", "c1", "c2", "c3", "gemm", "h2", "split", "attn", "bf16", "vendor"})

    import torch

    from . import audio, native, pack
    from .dims import CONFIG_DIMS

    dev = "cuda:0"
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    ctx = native.Context()
    reps = args.reps
    # bring the clocks up before the first timed kernel (about 0.3 s of matrix work)
    x = torch.randn(8192, 8192, device=dev, generator=g)
    for _ in range(20):
        x = torch.matmul(x, x).clamp_(-1.0, 1.0)
    torch.cuda.synchronize()
    del x

    if "copy" in groups:
        # practical ceiling of a 1:1 read/write stream, and the calibration
        # kernel for the FETCH_SIZE / WRITE_SIZE counters: a plain device copy
        # (torch's copy kernel) of 1.27 GB
        cs = torch.randn(496 * 801 * 801, device=dev, generator=g)
        cd = torch.empty_like(cs)
        _emit("copy_reference", _event_time(lambda: cd.copy_(cs), reps), gbytes=2 * cs.numel() * 4 / 1e9,
              shape="1.27 GB -> 1.27 GB", device=r"__amd_rocclr_copyBuffer", reps=reps)
        del cs, cd

    if "c1" in groups:
        rows, dim = 49662, 384
        gamma = 1 + 0.02 * torch.randn(dim, device=dev, generator=g)
        n = _sets_for(2 * rows * dim * 4)
        xs = [torch.randn(rows, dim, device=dev, generator=g) for _ in range(n)]
        ys = [torch.empty_like(x) for x in xs]
        _emit("rmsnorm", _event_time_sets([lambda x=x, y=y: ctx.rmsnorm(x, gamma, y, rows, dim)
                                           for x, y in zip(xs, ys)], reps),
              gbytes=2 * rows * dim * 4 / 1e9, shape=f"[49662,384], {n} buffer sets", device=r"rmsnorm_kernel", reps=reps)
        del xs, ys
        srows, slen = 496 * 801, 801
        n = _sets_for(2 * srows * slen * 4)
        ss = [torch.randn(srows, slen, device=dev, generator=g) for _ in range(n)]
        sos = [torch.empty_like(t) for t in ss]
        _emit("softmax_rows", _event_time_sets([lambda a=a, b=b: ctx.softmax_rows(a, b, srows, slen)
                                                for a, b in zip(ss, sos)], reps),
              gbytes=2 * srows * slen * 4 / 1e9, shape=f"[496,801,801], {n} buffer sets", device=r"softmax_rows_kernel", reps=reps)
        del ss, sos
        for b, length in ((62, 801), (801, 62)):
            n = _sets_for(2 * b * 8 * length * 64 * 4)
            rs = [torch.randn(b, 8, length, 64, device=dev, generator=g) for _ in range(n)]
            _emit("rope", _event_time_sets([lambda r=r: ctx.rope_bhld(r, b * 8, length) for r in rs], reps),
                  gbytes=2 * rs[0].numel() * 4 / 1e9, shape=f"[{b},8,{length},64], {n} buffer sets",
                  device=r"rope_bhld_kernel", reps=reps)
            del rs
        n = _sets_for(rows * (3072 + 1536) * 4)
        gis = [torch.randn(rows, 3072, device=dev, generator=g) for _ in range(n)]
        gos = [torch.empty(rows, 1536, device=dev) for _ in range(n)]
        _emit("geglu", _event_time_sets([lambda a=a, b=b: ctx.geglu(a, b, rows, 1536) for a, b in zip(gis, gos)], reps),
              gbytes=rows * (3072 + 1536) * 4 / 1e9, shape=f"[49662,3072]->[49662,1536], {n} buffer sets",
              device=r"geglu_kernel", reps=reps)
        del gis, gos
        n = _sets_for(3 * rows * dim * 4)
        xs = [torch.randn(rows, dim, device=dev, generator=g) for _ in range(n)]
        rs = [torch.randn(rows, dim, device=dev, generator=g) for _ in range(n)]
        _emit("residual_add", _event_time_sets([lambda x=x, r=r: ctx.residual_add(x, r, rows * dim)
                                                for x, r in zip(xs, rs)], reps),
              gbytes=3 * rows * dim * 4 / 1e9, shape=f"[49662,384], {n} buffer sets", device=r"residual_add_kernel", reps=reps)
        del xs, rs

    if "gemm" in groups:
        # the transformer GEMMs of one 8-window pass (M = 8 * 801 * 62 tokens)
        # on the fp32 MFMA instruction
        M = 8 * 801 * 62
        shapes = (("gemm_qkv_gates", 384, 1568, native.EPI_STORE, 1568),
                  ("gemm_out_residual", 512, 384, native.EPI_RESIDUAL, 384),
                  ("gemm_ff1_geglu", 384, 3072, native.EPI_GEGLU, 1536),
                  ("gemm_ff2_residual", 1536, 384, native.EPI_RESIDUAL, 384))
        for name, K, N, epi, ocols in shapes:
            a = torch.randn(M, K, device=dev, generator=g)
            w = 0.05 * torch.randn(N, K, device=dev, generator=g)
            b = torch.randn(N, device=dev, generator=g)
            c = torch.zeros(M, ocols, device=dev)
            r = max(3, reps // 4)
            _emit(name, _event_time(lambda: ctx.gemm(a, w, c, M, N, K, bias=b, epilogue=epi), r),
                  gflop=2.0 * M * K * N / 1e9, shape=f"M={M} K={K} N={N}", device=r"gemm_f32_kernel", reps=r)
            del a, w, b, c

    if "split" in groups:
        # the same four GEMMs in fp32 accuracy on the bf16 matrix cores (three
        # bf16 pieces per fp32 operand, six piece products): algorithmic fp32
        # FLOPs against the fp32 MFMA peak, and the matrix-core work (6x)
        # against the bf16 peak
        M = 8 * 801 * 62
        shapes = (("gemm_split_qkv_gates", 384, 1568, native.EPI_STORE, 1568),
                  ("gemm_split_out_residual", 512, 384, native.EPI_RESIDUAL, 384),
                  ("gemm_split_ff1_geglu", 384, 3072, native.EPI_GEGLU, 1536),
                  ("gemm_split_ff2_residual", 1536, 384, native.EPI_RESIDUAL, 384))
        for name, K, N, epi, ocols in shapes:
            a = torch.randn(M, K, device=dev, generator=g)
            w = 0.05 * torch.randn(N, K, device=dev, generator=g)
            ws = torch.empty(ctx.split_bytes(N, K) // 2, dtype=torch.bfloat16, device=dev)
            ctx.split_weights(w, ws, N, K)
            b = torch.randn(N, device=dev, generator=g)
            c = torch.zeros(M, ocols, device=dev)
            r = max(3, reps // 4)
            t = _event_time(lambda: ctx.gemm_split(a, ws, c, M, N, K, bias=b, epilogue=epi), r)
            _emit(name, t, gflop=2.0 * M * K * N / 1e9, shape=f"M={M} K={K} N={N}", peak_tflops=BF16_TFLOPS,
                  mc_products=6, device=r"gemm_split_kernel", reps=r)
            del a, w, ws, b, c

    if "h2" in groups or "ff1" in groups:
        # the same four GEMMs as the default fp32 path runs them: fp16 two-piece
        # splits (three products); QKV takes the residual stream itself with
        # its pre-norm inside the GEMM (row norm, the gain folded into the
        # weight's pieces, bound max|x|), FFN up reads A as RMSNorm h2 rows,
        # the others split fp32 A bounded by its maximum, FFN down also
        # raising the stream's bound for the next QKV GEMM
        M = 8 * 801 * 62
        shapes = (("gemm_h2_qkv_gates", 384, 1568, native.EPI_STORE, 1568),
                  ("gemm_h2_out_residual", 512, 384, native.EPI_RESIDUAL, 384),
                  ("gemm_h2_ff1_geglu", 384, 3072, native.EPI_GEGLU, 1536),
                  ("gemm_h2_ff2_residual", 1536, 384, native.EPI_RESIDUAL, 384))
        if "h2" not in groups:
            shapes = shapes[2:3]  # the dominant kernel alone (counter runs)
        for name, K, N, epi, ocols in shapes:
            a = torch.randn(M, K, device=dev, generator=g)
            w = 0.05 * torch.randn(N, K, device=dev, generator=g)
            wp = torch.empty(ctx.h2_bytes(N, K) // 2, dtype=torch.float16, device=dev)
            gamma = 1.0 + 0.02 * torch.randn(K, device=dev, generator=g)
            b = torch.randn(N, device=dev, generator=g)
            c = torch.zeros(M, ocols, device=dev)
            dbound = a.abs().max().reshape(1)
            if name == "gemm_h2_qkv_gates":
                ctx.split_weights_h2((w * gamma).contiguous(), wp, N, K)
                call = lambda: ctx.gemm_h2_ex(a, wp, c, M, N, K, dbound, bias=b, epilogue=epi, row_norm=True)
            elif name == "gemm_h2_ff1_geglu":
                ctx.split_weights_h2(w, wp, N, K)
                bnd = torch.zeros(2, device=dev)
                ctx.operand_bounds(gamma, K, bnd)
                ah = torch.empty_like(a)
                ctx.rmsnorm_h2(a, gamma, bnd, ah, M, K)
                bound = float(bnd[0])
                call = lambda: ctx.gemm_h2(ah, wp, c, M, N, K, bias=b, epilogue=epi, a_bound=bound, a_rows=True)
            elif name == "gemm_h2_ff2_residual":
                ctx.split_weights_h2(w, wp, N, K)
                amax = torch.zeros(1, device=dev)
                call = lambda: ctx.gemm_h2_ex(a, wp, c, M, N, K, dbound, bias=b, epilogue=epi, amax=amax)
            else:
                ctx.split_weights_h2(w, wp, N, K)
                call = lambda: ctx.gemm_h2_ex(a, wp, c, M, N, K, dbound, bias=b, epilogue=epi)
            r = max(3, reps // 4)
            t = _event_time(call, r)
            _emit(name, t, gflop=2.0 * M * K * N / 1e9, shape=f"M={M} K={K} N={N}", peak_tflops=FP16_TFLOPS,
                  mc_products=3, device=r"gemm_h2_kernel", reps=r)
            del a, w, wp, b, c

    if "bf16" in groups:
        # the same four GEMMs on bf16 matrix-core operands, with the operand
        # types of the bf16 pipeline: bf16 activations in, bf16 projections and
        # FFN hidden layer out, fp32 residual stream
        M = 8 * 801 * 62
        for name, K, N, epi, ocols, c16 in (("gemm_bf16_qkv_gates", 384, 1568, native.EPI_STORE, 1568, True),
                                            ("gemm_bf16_out_residual", 512, 384, native.EPI_RESIDUAL, 384, False),
                                            ("gemm_bf16_ff1_geglu", 384, 3072, native.EPI_GEGLU, 1536, True),
                                            ("gemm_bf16_ff2_residual", 1536, 384, native.EPI_RESIDUAL, 384, False)):
            a = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
            w = 0.05 * torch.randn(N, K, device=dev, generator=g)
            wh = torch.empty(N, K, dtype=torch.bfloat16, device=dev)
            ctx.to_bf16(w, wh, N, K, K)
            b = torch.randn(N, device=dev, generator=g)
            c = torch.zeros(M, ocols, device=dev, dtype=torch.bfloat16 if c16 else torch.float32)
            flags = native.BF16_A | (native.BF16_C if c16 else 0)
            r = max(3, reps // 4)
            _emit(name, _event_time(lambda: ctx.gemm_bf16(a, wh, c, M, N, K, K, bias=b, epilogue=epi, flags=flags), r),
                  gflop=2.0 * M * K * N / 1e9, shape=f"M={M} K={K} N={N}", peak_tflops=BF16_TFLOPS,
                  device=r"gemm_bf16_(dma_)?kernel", reps=r)
            del a, w, wh, b, c

    if "vendor" in groups:
        # reference point, not part of the library: the vendor GEMM (torch.matmul
        # on hipBLASLt) on the same four shapes with a plain store -- no bias,
        # no epilogue, C as wide as N (the fused kernels above add the bias,
        # the GELU-GLU or the residual read-modify-write)
        M = 8 * 801 * 62
        for dt, tag, peak in ((torch.bfloat16, "bf16", BF16_TFLOPS), (torch.float32, "fp32", FP32_TFLOPS)):
            for name, K, N in (("qkv_gates", 384, 1568), ("out", 512, 384), ("ff1", 384, 3072), ("ff2", 1536, 384)):
                a = torch.randn(M, K, device=dev, generator=g).to(dt)
                w = (0.05 * torch.randn(N, K, device=dev, generator=g)).to(dt)
                c = torch.empty(M, N, device=dev, dtype=dt)
                r = max(3, reps // 4)
                _emit(f"vendor_{tag}_{name}", _event_time(lambda: torch.matmul(a, w.t(), out=c), r),
                      gflop=2.0 * M * K * N / 1e9, shape=f"M={M} K={K} N={N}", peak_tflops=peak,
                      device=r"^Cijk_", reps=r)
                del a, w, c

    if "attn" in groups:
        # the two attention shapes of one 8-window pass; the fp16 two-piece
        # calls also compute max|qkv| (absmax kernels, not counted in the
        # rocprof pairing of the attention kernel itself)
        r = max(3, reps // 4)
        for S, L in ((8 * 62, 801), (8 * 801, 62)):
            qkv = torch.randn(S * L, 3 * 512, device=dev, generator=g)
            o = torch.empty(S * L, 512, device=dev)
            gf = 4.0 * S * 8 * L * L * 64 / 1e9
            long = L > 64
            _emit("attention_fp32", _event_time(lambda: ctx.attention(qkv, o, S, L, 8, True), r), gflop=gf,
                  shape=f"S={S} L={L} H=8", reps=r,
                  device=r"vh::attention_kernel<4" if long else r"attention_short_kernel<")
            if long:
                _emit("attention_split", _event_time(lambda: ctx.attention(qkv, o, S, L, 8, True, split=True), r),
                      gflop=gf, shape=f"S={S} L={L} H=8", peak_tflops=BF16_TFLOPS, mc_products=6,
                      device=r"attention_split_kernel", reps=r)
            # the default path's kernels: fp16 two-piece products; the band
            # axis (15.5 FLOP per byte) is priced against HBM: q, k, v read
            # and the output written once
            t = _event_time(lambda: ctx.attention(qkv, o, S, L, 8, True, h2=True), r)
            if long:
                _emit("attention_h2", t, gflop=gf, shape=f"S={S} L={L} H=8", peak_tflops=FP16_TFLOPS, mc_products=3,
                      reps=r, device=r"attention_h2_kernel")
            else:
                _emit("attention_short_h2", t, gbytes=S * L * 4 * 512 * 4 / 1e9, shape=f"S={S} L={L} H=8", reps=r,
                      device=r"attention_short_h2_kernel", extra={"algorithmic_GFLOP": round(gf, 2)})
            del qkv, o
        # the default path's band axis: the pre-norm q, k, v and gate projection
        # and the attention in one kernel, driven through a one-layer block at
        # the pass's band-axis shape (live ms: the whole block; rocprof ms: the
        # fused kernel alone)
        d1 = CONFIG_DIMS.with_depth(1)
        bmodel = native.Model(ctx, d1, pack.synthetic_pack(d1, 3))
        S, L = 8 * 801, 62
        xb = torch.randn(S * L, d1.dim, device=dev, generator=g)
        gf = (2.0 * S * L * d1.dim * 3 * 512 + 4.0 * S * 8 * L * L * 64) / 1e9
        _emit("band_attention_fused", _event_time(lambda: bmodel.transformer(0, 1, xb, S, L), r), gflop=gf,
              shape=f"S={S} L={L} H=8, dim {d1.dim}", peak_tflops=FP16_TFLOPS, mc_products=3,
              device=r"band_attention_fused_kernel", reps=r)
        del xb
        bmodel.close()

    if "c2" in groups or "c3" in groups:
        d = CONFIG_DIMS.with_depth(1)
        blob = pack.synthetic_pack(d, 2)
        model = native.Model(ctx, d, blob)
        T, B, D = 801, 62, 384
        tokens = T * B
        lin = 2.0 * tokens * (D * 1536 + D * 8 + 512 * D + D * 3072 + 1536 * D) / 1e9
        if "c2" in groups:
            xt = torch.randn(B, T, D, device=dev, generator=g)
            att_t = 4.0 * B * 8 * T * T * 64 / 1e9
            _emit("time_transformer", _event_time(lambda: model.transformer(0, 0, xt, B, T), max(3, reps // 4)),
                  gflop=lin + att_t, shape="62 seq x 801, dim 384", peak_tflops=FP16_TFLOPS, mc_products=3)
            xb = torch.randn(T, B, D, device=dev, generator=g)
            att_b = 4.0 * T * 8 * B * B * 64 / 1e9
            _emit("band_transformer", _event_time(lambda: model.transformer(0, 1, xb, T, B), max(3, reps // 4)),
                  gflop=lin + att_b, shape="801 seq x 62, dim 384", peak_tflops=FP16_TFLOPS, mc_products=3)
            del xt, xb
        if "c3" in groups:
            x = torch.from_numpy(audio.sine_mix(60.0, 60)).to(dev)
            length = x.shape[1]
            Tf = d.frames(length)
            # spectra in the pipeline's frame-major layout [C][T][F][2]
            fm = native.SPEC_FRAME_MAJOR
            src = torch.empty(d.channels, Tf, d.freq_bins, 2, device=dev)
            _emit("stft", _event_time(lambda: model.stft(x, length, src, fm), reps),
                  gbytes=(x.numel() + src.numel()) * 4 / 1e9, shape=f"60 s, T={Tf}", device=r"stft_kernel", reps=reps)
            mask = torch.randn_like(src)
            out = torch.empty_like(x)
            _emit("istft", _event_time(lambda: model.istft(src, mask, length, out, fm), reps),
                  gbytes=(2 * src.numel() + out.numel()) * 4 / 1e9, shape=f"60 s, T={Tf}",
                  device=r"istft_frames_kernel|ola_kernel", per_call=2, reps=reps)
            seq = torch.empty(d.bands, Tf, D, device=dev)
            _emit("band_split", _event_time(lambda: model.band_split(src, Tf, seq, fm), reps),
                  gflop=2.0 * Tf * sum(d.input_dims()) * D / 1e9, shape=f"T={Tf}, 62 bands",
                  device=r"band_gather_norm_kernel|gemm_f32_batched_kernel", per_call=2, reps=reps)
            feats = torch.randn(Tf, d.bands, D, device=dev, generator=g)
            mout = torch.empty_like(src)
            gf = 2.0 * Tf * (d.bands * D * d.mask_hidden + d.mask_hidden * 2 * sum(d.input_dims())) / 1e9
            r = max(3, reps // 4)
            _emit("mask_estimator", _event_time(lambda: model.mask_estimate(feats, Tf, mout, fm), r),
                  gflop=gf, shape=f"T={Tf}, 62 bands", peak_tflops=FP16_TFLOPS, mc_products=3,
                  device=r"gemm_h2_batched_kernel|mask_glu_scatter_kernel", per_call=3, reps=r)
        model.close()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
