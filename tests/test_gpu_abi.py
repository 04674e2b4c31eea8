"""The native_gpu.h drop-in boundary on the GPU.

1. The provider driven through its C-ABI exactly as the reference host drives
   it (native/vocalarc_separation.c:1356-1406), checked against the oracle.
2. The reference C11 host itself (compiled from the reference sources into
   oracle/_ref and linked against lib/libvocalarc_hip.so) checked against the
   reference CPU executable on the same pack and WAV: the fp32 parity bar,
   max |delta| <= 1e-4 and SNR >= 80 dB on the vocals and instrumental.
"""

import ctypes
import json
import os
import subprocess
import tempfile
from pathlib import Path

import numpy as np
import pytest

from helpers import assert_close, gpu_available, snr_db

pytestmark = pytest.mark.gpu

if gpu_available():
    import oracle as O
    from vocalarc_hip import audio, native, pack
    from vocalarc_hip.dims import REFERENCE_DIMS as RD

_F = ctypes.POINTER(ctypes.c_float)


class TW(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("gamma", "qkv", "gate_weight", "gate_bias", "out_weight", "ff_gamma",
                                             "ff1_weight", "ff1_bias", "ff2_weight", "ff2_bias")]


class MB(ctypes.Structure):
    _fields_ = [("first_weight", ctypes.c_void_p), ("first_bias", ctypes.c_void_p),
                ("second_weight", ctypes.c_void_p), ("second_bias", ctypes.c_void_p),
                ("input_dim", ctypes.c_int), ("first_frequency", ctypes.c_int)]


def _weights(views, layer, axis):
    p = f"layers.{layer}.{axis}."
    return TW(*[views[p + n].ctypes.data for n in ("gamma", "qkv", "gate_weight", "gate_bias", "out_weight",
                                                    "ff_gamma", "ff1_weight", "ff1_bias", "ff2_weight", "ff2_bias")])


@pytest.fixture(scope="module")
def provider():
    if not gpu_available():
        pytest.skip("no GPU")
    L = native.lib()
    g = L.native_gpu_create()
    assert g, "native_gpu_create returned NULL on a GPU box"
    yield L, g
    L.native_gpu_destroy(g)


@pytest.fixture(scope="module")
def views(ref_pack):
    return pack.tensor_views(RD, ref_pack)


def test_backend_strings(provider):
    L, g = provider
    assert L.native_gpu_backend(g) == b"native-hip-fused"
    dev = L.native_gpu_device(g).decode()
    assert dev and '"' not in dev and "\\" not in dev
    assert L.native_gpu_backend(None) == b"native-cpu"
    assert L.native_gpu_device(None) == b"none"
    assert L.native_gpu_uses_full_batches(g) == 1
    assert L.native_gpu_can_use_full_batches(g, 87) == 1
    assert L.native_gpu_can_use_full_batches(g, 0) == 0


def test_full_batch_admission(provider, monkeypatch):
    """native_gpu_can_use_full_batches: the reference policy (the resident
    working set below 3/5 of free device memory, VOCALARC_GPU_FULL_BATCHES
    0/false/off declines; native/native_gpu_cuda.cu:859-879) plus the decline
    when the host's full-batch scratch, max(bands, frames)^2 tokens of
    dim + qkv + inner + heads floats (native/vocalarc_separation.c:1262-1276,
    1576-1582), would exceed half of host memory."""
    L, g = provider
    assert L.native_gpu_can_use_full_batches(g, 862) == 1  # config 0 (10 s)
    # 5 minutes whole-file: 25840^2 tokens of 2312 floats = 6.2 TB of host scratch
    assert L.native_gpu_can_use_full_batches(g, 25840) == 0
    for v in ("0", "false", "off"):
        monkeypatch.setenv("VOCALARC_GPU_FULL_BATCHES", v)
        assert L.native_gpu_can_use_full_batches(g, 862) == 0
    monkeypatch.setenv("VOCALARC_GPU_FULL_BATCHES", "1")
    assert L.native_gpu_can_use_full_batches(g, 862) == 1
    monkeypatch.delenv("VOCALARC_GPU_FULL_BATCHES")
    # the host-scratch boundary: side^2 * 2312 * 4 B = half of physical memory
    ram = os.sysconf("SC_PHYS_PAGES") * os.sysconf("SC_PAGE_SIZE")
    per_token = (RD.dim + 3 * RD.heads * RD.dim_head + RD.heads * RD.dim_head + RD.heads) * 4
    assert per_token == 2312 * 4
    side = (0.5 * ram / per_token) ** 0.5
    below, above = int(side) - 1, int(side) + 2
    assert below > RD.bands
    print(f"admission: host memory {ram / 2**30:.0f} GiB, host-scratch boundary at {side:.0f} frames")
    assert L.native_gpu_can_use_full_batches(g, above) == 0
    assert L.native_gpu_can_use_full_batches(g, below) == 1


def test_resident_path_matches_oracle(provider, views, ref_pack):
    """begin -> 16 x {time, transpose, band, transpose} -> mask, as the host
    calls it, vs the oracle's stack + final norm + mask estimator."""
    L, g = provider
    om = O.Model(RD, ref_pack)
    x = audio.sine_mix(0.25, 21)
    src = O.stft(RD, x)
    T = src.shape[2]
    seq = om.band_split(src)  # [B][T][D]
    # oracle stack on the same input
    feats = seq.transpose(1, 0, 2).copy()
    cur = seq.copy()
    for layer in range(RD.depth):
        cur = om.transformer(layer, 0, cur, RD.bands, T)
        feats = cur.transpose(1, 0, 2).copy()
        feats = om.transformer(layer, 1, feats, T, RD.bands)
        cur = feats.transpose(1, 0, 2).copy()
    normed = O.rms_norm(feats.reshape(-1, RD.dim), views["final_gamma"]).reshape(feats.shape)
    ref_mask = om.mask_estimate(normed)

    assert L.native_gpu_resident_begin(g, RD.bands, T, seq.ctypes.data) == 1
    for layer in range(RD.depth):
        tw, fw = _weights(views, layer, 0), _weights(views, layer, 1)
        assert L.native_gpu_resident_transformer(g, RD.bands, T, ctypes.byref(tw)) == 1
        assert L.native_gpu_resident_transpose(g, RD.bands, T) == 1
        assert L.native_gpu_resident_transformer(g, T, RD.bands, ctypes.byref(fw)) == 1
        if layer + 1 < RD.depth:
            assert L.native_gpu_resident_transpose(g, T, RD.bands) == 1
    bands = (MB * RD.bands)()
    for b, f0 in enumerate(RD.first_frequencies()):
        bands[b] = MB(views[f"masks.{b}.first_weight"].ctypes.data, views[f"masks.{b}.first_bias"].ctypes.data,
                      views[f"masks.{b}.second_weight"].ctypes.data, views[f"masks.{b}.second_bias"].ctypes.data,
                      RD.input_dims()[b], f0)
    mask = np.zeros_like(ref_mask)
    assert L.native_gpu_resident_mask(g, T, views["final_gamma"].ctypes.data, mask.ctypes.data, bands, RD.bands) == 1
    assert_close(ref_mask, mask, rtol=1e-3, atol=1e-5, min_snr=80, what="resident mask")
    # residency ended with the mask
    assert L.native_gpu_resident_transpose(g, T, RD.bands) == 0


def test_resident_transpose_and_end_roundtrip(provider, rng):
    """transpose is a logical flip; end returns the tensor in the current
    logical order, bit for bit."""
    L, g = provider
    S, Ln = 90, 17
    x = rng.standard_normal((S, Ln, RD.dim), dtype=np.float32)
    out = np.empty_like(x)
    assert L.native_gpu_resident_begin(g, S, Ln, x.ctypes.data) == 1
    assert L.native_gpu_resident_transpose(g, S, Ln) == 1
    o2 = np.empty((Ln, S, RD.dim), np.float32)
    assert L.native_gpu_resident_end(g, o2.ctypes.data) == 1
    assert np.array_equal(o2, x.transpose(1, 0, 2))
    # two transposes give back the original
    assert L.native_gpu_resident_begin(g, S, Ln, x.ctypes.data) == 1
    assert L.native_gpu_resident_transpose(g, S, Ln) == 1
    assert L.native_gpu_resident_transpose(g, Ln, S) == 1
    assert L.native_gpu_resident_end(g, out.ctypes.data) == 1
    assert np.array_equal(out, x)
    # a stale residency is reset by the next begin
    assert L.native_gpu_resident_begin(g, S, Ln, x.ctypes.data) == 1
    assert L.native_gpu_resident_begin(g, S, Ln, x.ctypes.data) == 1
    assert L.native_gpu_resident_end(g, out.ctypes.data) == 1
    # token-count mismatch is refused
    assert L.native_gpu_resident_begin(g, S, Ln, x.ctypes.data) == 1
    assert L.native_gpu_resident_transformer(g, S, Ln + 1, None) == 0
    assert L.native_gpu_resident_end(g, out.ctypes.data) == 1


def test_nonresident_transformer(provider, views, ref_pack, rng):
    L, g = provider
    om = O.Model(RD, ref_pack)
    S, Ln = 16, 40
    x = rng.standard_normal((S, Ln, RD.dim), dtype=np.float32)
    ref = om.transformer(3, 0, x, S, Ln)
    data = x.copy()
    w = _weights(views, 3, 0)
    assert L.native_gpu_transformer(g, S, Ln, data.ctypes.data, None, None, None, None, ctypes.byref(w)) == 1
    assert_close(ref, data, rtol=1e-4, atol=1e-4, min_snr=100, what="native_gpu_transformer")


def test_matmul(provider, views, rng, monkeypatch):
    L, g = provider
    monkeypatch.setenv("VOCALARC_GPU_MIN_WORK", "0")
    for b in (0, 60, 89):
        in_dim = RD.input_dims()[b]
        x = rng.standard_normal((37, in_dim), dtype=np.float32)
        w, bias = views[f"bands.{b}.weight"], views[f"bands.{b}.bias"]
        ref = O.matmul(x, w, RD.dim, bias)
        out = np.empty((37, RD.dim), np.float32)
        assert L.native_gpu_matmul(g, 37, in_dim, RD.dim, x.ctypes.data, w.ctypes.data, bias.ctypes.data,
                                   out.ctypes.data) == 1
        assert_close(ref, out, rtol=2e-5, atol=2e-6, what=f"matmul band {b}")
    # inputs beyond the fp16 two-piece scale range (max |x| > 1e30) take the
    # fp32 MFMA GEMM instead of overflowing a piece
    b = 60
    in_dim = RD.input_dims()[b]
    assert in_dim % 16 == 0  # a width the two-piece GEMM would otherwise serve
    x = rng.standard_normal((37, in_dim), dtype=np.float32) * np.float32(1e33)
    w, bias = views[f"bands.{b}.weight"], views[f"bands.{b}.bias"]
    ref = O.matmul(x, w, RD.dim, bias)
    out = np.empty((37, RD.dim), np.float32)
    assert L.native_gpu_matmul(g, 37, in_dim, RD.dim, x.ctypes.data, w.ctypes.data, bias.ctypes.data,
                               out.ctypes.data) == 1
    assert np.all(np.isfinite(out))
    assert_close(ref, out, rtol=2e-5, atol=2e27, what="matmul beyond the scale range")
    monkeypatch.setenv("VOCALARC_GPU_MIN_WORK", str(1 << 40))
    assert L.native_gpu_matmul(g, 37, 8, RD.dim, x.ctypes.data, w.ctypes.data, None, out.ctypes.data) == 0


# ---------------------------------------------------------------- host path

# Input length of the host-path tests: 10 s, the config-0 case (T = 862
# frames; the reference CPU executable takes about 20 s of it on 16 cores),
# unless VOCALARC_HOST_SECONDS asks for another (1 s is the reference's
# published benchmark length).
HOST_SECONDS = float(os.environ.get("VOCALARC_HOST_SECONDS", "10.0"))
HOST_THREADS = int(os.environ.get("VOCALARC_HOST_THREADS", str(min(16, os.cpu_count() or 1))))


def _run_host(exe, pack_path, wav, tmp, tag, env=None, repetitions=1):
    """Run the host's JSONL protocol; with repetitions > 1 the first request is
    a warm-up and the response carries the median inferenceMs of the rest
    (native/scripts/benchmark.py:135-161 protocol)."""
    v, i = tmp / f"{tag}-v.wav", tmp / f"{tag}-i.wav"
    resp = O.run_reference(exe, pack_path, wav, v, i, threads=HOST_THREADS, env_extra=env, repetitions=repetitions,
                           timeout=3600)
    sep = [r for r in resp if r.get("type") == "separated"]
    assert sep and all(r["ok"] for r in sep), resp
    res = dict(sep[-1])
    timed = sep[1:] if len(sep) > 1 else sep
    res["inferenceMs"] = float(np.median([r["inferenceMs"] for r in timed]))
    return res, audio.read_wav_float(v)[0], audio.read_wav_float(i)[0]


@pytest.fixture(scope="module")
def host_setup(ref_pack):
    if not gpu_available():
        pytest.skip("no GPU")
    if not (O.REF_EXE.exists() and O.REF_GPU_EXE.exists()):
        pytest.skip("reference executables not built (make -C oracle ref gpu-host)")
    tmp = Path(tempfile.mkdtemp(prefix="vocalarc-host-"))
    pack_path = tmp / "model.f32"
    pack.write_pack(pack_path, ref_pack)
    wav = tmp / "in.wav"
    # config-0 recipe: 6 sines (80-4000 Hz, a ~ U(0.02, 0.1)) + N(0, 0.01^2) per channel
    audio.write_wav_float(wav, audio.sine_mix(HOST_SECONDS, 2026))
    cpu = _run_host(O.REF_EXE, pack_path, wav, tmp, "cpu")
    return tmp, pack_path, wav, cpu


def test_reference_host_with_hip_provider(host_setup):
    tmp, pack_path, wav, (cpu_resp, cpu_v, cpu_i) = host_setup
    resp, v, i = _run_host(O.REF_GPU_EXE, pack_path, wav, tmp, "gpu", repetitions=4)
    assert resp["backend"] == "native-hip-fused"
    assert cpu_resp["backend"] == "native-cpu"
    for ref, out, name in ((cpu_v, v, "vocals"), (cpu_i, i, "instrumental")):
        err = float(np.max(np.abs(out.astype(np.float64) - ref)))
        assert err <= 1e-4, (name, err)
        assert snr_db(ref, out) >= 80, (name, snr_db(ref, out))
    secs = resp["seconds"]
    print(f"host path {secs:.1f} s ({resp['frames']} frames): reference CPU executable {cpu_resp['inferenceMs']:.1f} ms "
          f"({HOST_THREADS} threads, RTF {secs / cpu_resp['inferenceMs'] * 1e3:.3f}); with the HIP provider "
          f"{resp['inferenceMs']:.1f} ms median of 3 (RTF {secs / resp['inferenceMs'] * 1e3:.2f}); vocals max|d| "
          f"{float(np.max(np.abs(v.astype(np.float64) - cpu_v))):.2e} SNR {snr_db(cpu_v, v):.1f} dB; "
          f"instrumental SNR {snr_db(cpu_i, i):.1f} dB")


def test_reference_host_nonresident_groups(host_setup):
    """VOCALARC_GPU_FULL_BATCHES=0: the host keeps its bounded groups and calls
    native_gpu_transformer per group (native/vocalarc_separation.c:846)."""
    tmp, pack_path, wav, (_, cpu_v, _) = host_setup
    resp, v, _ = _run_host(O.REF_GPU_EXE, pack_path, wav, tmp, "gpu-groups", env={"VOCALARC_GPU_FULL_BATCHES": "0"})
    assert resp["backend"] == "native-hip-fused"
    assert float(np.max(np.abs(v.astype(np.float64) - cpu_v))) <= 1e-4
    assert snr_db(cpu_v, v) >= 80


def test_reference_host_fp32_mfma_products(host_setup):
    """VOCALARC_GPU_SPLIT=0: every product of the provider (linears and
    attention) on the fp32 MFMA instruction; the same parity bar, and close to
    the default fp16 two-piece output."""
    tmp, pack_path, wav, (_, cpu_v, _) = host_setup
    resp, v, _ = _run_host(O.REF_GPU_EXE, pack_path, wav, tmp, "gpu-fp32", env={"VOCALARC_GPU_SPLIT": "0"})
    assert resp["backend"] == "native-hip-fused"
    assert float(np.max(np.abs(v.astype(np.float64) - cpu_v))) <= 1e-4
    assert snr_db(cpu_v, v) >= 80
    _, v_default, _ = _run_host(O.REF_GPU_EXE, pack_path, wav, tmp, "gpu-default")
    print(f"host path, fp32 MFMA products vs default: SNR {snr_db(v_default, v):.1f} dB")
    assert snr_db(v_default, v) >= 100


def test_reference_host_gpu_off_is_cpu_path(host_setup):
    """VOCALARC_GPU=off: no provider; the gpu executable is the CPU path."""
    tmp, pack_path, wav, (_, cpu_v, _) = host_setup
    resp, v, _ = _run_host(O.REF_GPU_EXE, pack_path, wav, tmp, "gpu-off", env={"VOCALARC_GPU": "off"})
    assert resp["backend"] == "native-cpu"
    assert np.array_equal(v, cpu_v)


def test_embedded_pack_host(host_setup):
    """The HIP-linked host with the pack appended by the reference's embedder
    (native/embed_model.c: the pack, then 'VSCEMB01' and its u64 size) loads
    the model from its own executable when the model path does not exist
    (native/vocalarc_separation.c:334-375, 591-593; the protocol smoke of
    native/scripts/test_native.sh:8-18), reports the HIP backend, and
    separates bit for bit as the run that loads the same pack from a file."""
    tmp, pack_path, wav, _ = host_setup
    if not O.REF_EMBED.exists():
        pytest.skip("reference embedder not built (make -C oracle ref)")
    exe = tmp / "vocalarc-separation-gpu-embedded"
    subprocess.run([str(O.REF_EMBED), str(O.REF_GPU_EXE), str(pack_path), str(exe)], check=True, timeout=300)
    assert exe.stat().st_size == O.REF_GPU_EXE.stat().st_size + pack_path.stat().st_size + 16
    with open(exe, "rb") as f:
        f.seek(-16, os.SEEK_END)
        trailer = f.read()
    assert trailer[:8] == b"VSCEMB01" and int.from_bytes(trailer[8:], "little") == pack_path.stat().st_size

    libdir = str(native.LIB_PATH.parent)
    env = dict(os.environ, VOCALARC_NATIVE_MODEL=str(exe) + ".missing-model.f32",
               LD_LIBRARY_PATH=libdir + os.pathsep + os.environ.get("LD_LIBRARY_PATH", ""))
    v_emb = tmp / "embedded-v.wav"
    reqs = ['{"id":1,"type":"ping"}', '{"id":2,"type":"load"}',
            json.dumps({"id": 3, "type": "separate", "inputPath": str(wav), "vocalsPath": str(v_emb)}),
            '{"id":4,"type":"shutdown"}']
    proc = subprocess.run([str(exe), "--threads", str(HOST_THREADS)], input="\n".join(reqs) + "\n",
                          capture_output=True, text=True, env=env, timeout=1800)
    assert proc.returncode == 0, proc.stderr[-2000:]
    resp = {r["id"]: r for r in (json.loads(x) for x in proc.stdout.splitlines() if x.strip())}
    assert resp[1]["type"] == "pong" and resp[1]["runtime"]["backend"] == "native-hip-fused"
    assert resp[2]["type"] == "loaded" and resp[2]["backend"] == "native-hip-fused", resp[2]
    assert resp[2]["modelBytes"] == pack_path.stat().st_size
    assert resp[3]["ok"] and resp[3]["backend"] == "native-hip-fused", resp[3]
    assert resp[4]["type"] == "shutdown"

    _, v_file, _ = _run_host(O.REF_GPU_EXE, pack_path, wav, tmp, "gpu-file")
    v, _ = audio.read_wav_float(v_emb)
    assert np.array_equal(v, v_file)
