"""ctypes front end of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Loads oracle/liboracle.so (the C restatement in vocalarc_oracle.c) and, when
built, the reference artefacts in oracle/_ref/ (the reference CPU executable
and its AVX2 row kernels, compiled from the reference sources by
oracle/Makefile).  Only tests, the smoke entry point and the benchmark's CPU
baseline leg use this module.
"""

from __future__ import annotations

import ctypes
import json
import os
import subprocess
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
sys.path.insert(0, str(REPO / "karaoke-platform-sidecar-native_amd"))

from vocalarc_hip.dims import CDims, ModelDims, to_c  # noqa: E402

REF_DIR = HERE / "_ref"
REF_EXE = REF_DIR / "vocalarc-separation"
REF_GPU_EXE = REF_DIR / "vocalarc-separation-gpu"
REF_SIMD = REF_DIR / "libref_simd.so"
REF_EMBED = REF_DIR / "embed-model"

_F = ctypes.POINTER(ctypes.c_float)
_I64 = ctypes.c_int64


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


class _Layer(ctypes.Structure):
    _fields_ = [(n, _F) for n in ("gamma", "qkv", "gate_weight", "gate_bias", "out_weight",
                                  "ff_gamma", "ff1_weight", "ff1_bias", "ff2_weight", "ff2_bias")]


class _Model(ctypes.Structure):
    _fields_ = [("d", CDims), ("layers", ctypes.POINTER(_Layer)), ("bands", ctypes.c_void_p),
                ("final_gamma", _F), ("masks", ctypes.c_void_p)]


class _Dumps(ctypes.Structure):
    _fields_ = [(n, _F) for n in ("source", "band", "features0", "features1", "features_last", "mask")]


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
    if Path(os.environ.get("VOCALARC_REFERENCE", "/root/reference/native")).is_dir():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            build()
        L = ctypes.CDLL(str(path))
        L.or_fast_exp.restype = ctypes.c_float
        L.or_fast_exp.argtypes = [ctypes.c_float]
        L.or_dot.restype = ctypes.c_float
        L.or_model_parse.argtypes = [ctypes.POINTER(_Model), ctypes.POINTER(CDims), ctypes.c_void_p, ctypes.c_size_t]
        L.or_rms_norm.argtypes = [_I64, ctypes.c_int, _F, _F, _F]
        L.or_matmul.argtypes = [_I64, ctypes.c_int, ctypes.c_int, _F, _F, _F, _F]
        L.or_gelu.argtypes = [_I64, _F]
        L.or_geglu.argtypes = [_I64, ctypes.c_int, _F, _F]
        L.or_residual_add.argtypes = [_I64, _F, _F]
        L.or_softmax_rows.argtypes = [_I64, ctypes.c_int, _F, _F]
        L.or_rope_bhld.argtypes = [_I64, ctypes.c_int, ctypes.c_int, _F, _F, _F]
        L.or_rope_table.argtypes = [ctypes.c_int, ctypes.c_int, _F, _F]
        L.or_hann.argtypes = [ctypes.c_int, _F]
        L.or_transformer.argtypes = [ctypes.POINTER(CDims), ctypes.POINTER(_Layer), _F, ctypes.c_int, ctypes.c_int]
        L.or_attention.argtypes = [ctypes.POINTER(CDims), _F, _F, ctypes.c_int, ctypes.c_int]
        L.or_stft.argtypes = [ctypes.POINTER(CDims), _F, ctypes.c_int, ctypes.c_int, _F]
        L.or_istft.argtypes = [ctypes.POINTER(CDims), _F, _F, ctypes.c_int, ctypes.c_int, _F]
        L.or_band_split.argtypes = [ctypes.POINTER(_Model), _F, ctypes.c_int, _F]
        L.or_mask_estimate.argtypes = [ctypes.POINTER(_Model), _F, ctypes.c_int, _F]
        L.or_forward.argtypes = [ctypes.POINTER(_Model), _F, ctypes.c_int, _F, ctypes.POINTER(_Dumps)]
        L.or_forward_layers.argtypes = [ctypes.POINTER(_Model), _F, ctypes.c_int, ctypes.c_int, _F]
        L.or_separate_chunked.argtypes = [ctypes.POINTER(_Model), _F, ctypes.c_int, ctypes.c_int, ctypes.c_int, _F]
        L.or_chunk_count.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.or_chunk_weights.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _F]
        L.or_set_threads.argtypes = [ctypes.c_int]
        _lib = L
    return _lib


def set_threads(n: int) -> None:
    lib().or_set_threads(n)


# ---------------------------------------------------------------- kernels

def fast_exp(x: float) -> float:
    return lib().or_fast_exp(x)


def rms_norm(x: np.ndarray, gamma: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().or_rms_norm(x.shape[0], x.shape[1], _fp(x), _fp(np.ascontiguousarray(gamma, np.float32)), _fp(y))
    return y


def matmul(x: np.ndarray, packed_w: np.ndarray, out: int, bias: np.ndarray | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty((x.shape[0], out), np.float32)
    b = None if bias is None else _fp(np.ascontiguousarray(bias, np.float32))
    lib().or_matmul(x.shape[0], x.shape[1], out, _fp(x), _fp(np.ascontiguousarray(packed_w, np.float32)), b, _fp(y))
    return y


def gelu(x: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(x, np.float32).copy()
    lib().or_gelu(y.size, _fp(y))
    return y


def geglu(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    rows, w2 = x.shape
    y = np.empty((rows, w2 // 2), np.float32)
    lib().or_geglu(rows, w2 // 2, _fp(x), _fp(y))
    return y


def residual_add(x: np.ndarray, r: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(x, np.float32).copy()
    lib().or_residual_add(y.size, _fp(y), _fp(np.ascontiguousarray(r, np.float32)))
    return y


def softmax_rows(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    length = x.shape[-1]
    y = np.empty_like(x)
    lib().or_softmax_rows(x.size // length, length, _fp(x), _fp(y))
    return y


def rope_table(length: int, dim_head: int) -> tuple[np.ndarray, np.ndarray]:
    c = np.empty((length, dim_head // 2), np.float32)
    s = np.empty_like(c)
    lib().or_rope_table(length, dim_head, _fp(c), _fp(s))
    return c, s


def rope_bhld(x: np.ndarray) -> np.ndarray:
    """x: [..., L, Dh] rotated in a copy."""
    y = np.ascontiguousarray(x, np.float32).copy()
    L, Dh = y.shape[-2], y.shape[-1]
    c, s = rope_table(L, Dh)
    lib().or_rope_bhld(y.size // (L * Dh), L, Dh, _fp(y), _fp(c), _fp(s))
    return y


def hann(n_fft: int) -> np.ndarray:
    w = np.empty(n_fft, np.float32)
    lib().or_hann(n_fft, _fp(w))
    return w


def attention(d: ModelDims, qkv: np.ndarray, sequences: int, length: int) -> np.ndarray:
    qkv = np.ascontiguousarray(qkv, np.float32)
    out = np.empty((sequences * length, d.inner), np.float32)
    cd = to_c(d)
    lib().or_attention(ctypes.byref(cd), _fp(qkv), _fp(out), sequences, length)
    return out


def stft(d: ModelDims, audio: np.ndarray) -> np.ndarray:
    audio = np.ascontiguousarray(audio, np.float32)
    length = audio.shape[1]
    T = d.frames(length)
    src = np.empty((d.freq_bins, d.channels, T, 2), np.float32)
    cd = to_c(d)
    lib().or_stft(ctypes.byref(cd), _fp(audio), length, T, _fp(src))
    return src


def istft(d: ModelDims, source: np.ndarray, mask: np.ndarray, length: int) -> np.ndarray:
    T = source.shape[2]
    out = np.empty((d.channels, length), np.float32)
    cd = to_c(d)
    lib().or_istft(ctypes.byref(cd), _fp(np.ascontiguousarray(source, np.float32)),
                   _fp(np.ascontiguousarray(mask, np.float32)), length, T, _fp(out))
    return out


def chunk_count(length: int, chunk: int, step: int) -> int:
    return lib().or_chunk_count(length, chunk, step)


def chunk_weights(chunk: int, step: int, index: int, count: int) -> np.ndarray:
    w = np.empty(chunk, np.float32)
    lib().or_chunk_weights(chunk, step, index, count, _fp(w))
    return w


# ---------------------------------------------------------------- model

class Model:
    """A parsed pack.  Keeps the blob alive; tensors point into it."""

    def __init__(self, d: ModelDims, blob: np.ndarray):
        self.d = d
        self.blob = np.ascontiguousarray(blob, np.uint8)
        self.cd = to_c(d)
        self.m = _Model()
        ok = lib().or_model_parse(ctypes.byref(self.m), ctypes.byref(self.cd),
                                  self.blob.ctypes.data, self.blob.size)
        if not ok:
            raise ValueError("oracle could not parse the pack")

    def layer(self, layer: int, axis: int):
        return ctypes.pointer(self.m.layers[2 * layer + axis])

    def transformer(self, layer: int, axis: int, data: np.ndarray, sequences: int, length: int) -> np.ndarray:
        x = np.ascontiguousarray(data, np.float32).copy()
        lib().or_transformer(ctypes.byref(self.cd), self.layer(layer, axis), _fp(x), sequences, length)
        return x

    def band_split(self, source: np.ndarray) -> np.ndarray:
        T = source.shape[2]
        out = np.empty((self.d.bands, T, self.d.dim), np.float32)
        lib().or_band_split(ctypes.byref(self.m), _fp(np.ascontiguousarray(source, np.float32)), T, _fp(out))
        return out

    def mask_estimate(self, features_normed: np.ndarray) -> np.ndarray:
        T = features_normed.shape[0]
        out = np.empty((self.d.freq_bins, self.d.channels, T, 2), np.float32)
        lib().or_mask_estimate(ctypes.byref(self.m), _fp(np.ascontiguousarray(features_normed, np.float32)), T, _fp(out))
        return out

    def forward(self, audio: np.ndarray, dumps: bool = False):
        d = self.d
        audio = np.ascontiguousarray(audio, np.float32)
        length = audio.shape[1]
        T = d.frames(length)
        vocals = np.empty_like(audio)
        dd = None
        arrays = {}
        if dumps:
            spec = (d.freq_bins, d.channels, T, 2)
            arrays = {"source": np.empty(spec, np.float32), "band": np.empty((d.bands, T, d.dim), np.float32),
                      "features0": np.empty((T, d.bands, d.dim), np.float32),
                      "features1": np.empty((T, d.bands, d.dim), np.float32),
                      "features_last": np.empty((T, d.bands, d.dim), np.float32),
                      "mask": np.empty(spec, np.float32)}
            dd = _Dumps(**{k: _fp(v) for k, v in arrays.items()})
        ok = lib().or_forward(ctypes.byref(self.m), _fp(audio), length, _fp(vocals),
                              ctypes.byref(dd) if dd is not None else None)
        if not ok:
            raise RuntimeError("oracle forward failed")
        return (vocals, arrays) if dumps else vocals

    def forward_layers(self, audio: np.ndarray, layers: int) -> np.ndarray:
        d = self.d
        audio = np.ascontiguousarray(audio, np.float32)
        T = d.frames(audio.shape[1])
        feats = np.empty((T, d.bands, d.dim), np.float32)
        lib().or_forward_layers(ctypes.byref(self.m), _fp(audio), audio.shape[1], layers, _fp(feats))
        return feats

    def separate_chunked(self, audio: np.ndarray, chunk: int, step: int) -> np.ndarray:
        audio = np.ascontiguousarray(audio, np.float32)
        out = np.empty_like(audio)
        ok = lib().or_separate_chunked(ctypes.byref(self.m), _fp(audio), audio.shape[1], chunk, step, _fp(out))
        if not ok:
            raise RuntimeError("oracle chunked separation failed")
        return out


# ---------------------------------------------------------------- reference

def reference_available() -> bool:
    return REF_EXE.exists()


def run_reference(exe: Path, pack_path: Path, input_wav: Path, vocals_wav: Path,
                  instrumental_wav: Path | None = None, threads: int = 8, dump_prefix: str | None = None,
                  env_extra: dict | None = None, groups: tuple[int, int] | None = None,
                  repetitions: int = 1, timeout: float = 600) -> list[dict]:
    """Drive the reference JSONL protocol (native/vocalarc_separation.c:1537-1605)
    and return the parsed response lines of the `separate` requests."""
    env = dict(os.environ)
    if dump_prefix:
        env["VOCALARC_DEBUG_DUMP"] = dump_prefix
    if env_extra:
        env.update(env_extra)
    lines = ['{"id":1,"type":"ping"}', '{"id":2,"type":"load","modelPath":"%s"}' % pack_path]
    for r in range(repetitions):
        req = {"id": 10 + r, "type": "separate", "inputPath": str(input_wav), "vocalsPath": str(vocals_wav)}
        if instrumental_wav is not None:
            req["instrumentalPath"] = str(instrumental_wav)
        if groups is not None:
            req["timeBandGroup"], req["frequencyFrameGroup"] = groups
        lines.append(json.dumps(req))
    lines.append('{"id":99,"type":"shutdown"}')
    proc = subprocess.run([str(exe), "--model", str(pack_path), "--threads", str(threads)],
                          input="\n".join(lines) + "\n", capture_output=True, text=True, env=env,
                          timeout=timeout)
    responses = [json.loads(line) for line in proc.stdout.splitlines() if line.strip()]
    if proc.returncode != 0:
        raise RuntimeError(f"reference exited {proc.returncode}: {proc.stderr[-2000:]}")
    return responses


class RefSimd:
    """The reference AVX2 row kernels (native/native_simd.c) from oracle/_ref."""

    def __init__(self):
        L = ctypes.CDLL(str(REF_SIMD))
        L.vocalarc_dot_avx2.restype = ctypes.c_float
        L.vocalarc_dot_avx2.argtypes = [_F, _F, ctypes.c_int]
        L.vocalarc_axpy_avx2.argtypes = [_F, _F, ctypes.c_float]
        L.vocalarc_scale_head_avx2.argtypes = [_F, ctypes.c_float]
        L.vocalarc_matmul_row_avx2.argtypes = [_F, _F, _F, _F, ctypes.c_int, ctypes.c_int]
        L.vocalarc_rms_norm_row_avx2.argtypes = [_F, _F, _F, ctypes.c_int]
        self.L = L
