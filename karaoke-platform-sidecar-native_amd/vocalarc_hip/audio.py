"""Seeded audio, WAV I/O and waveform comparison.

WAV handling mirrors what the reference host reads and writes
(native/vocalarc_separation.c:1152-1237): PCM16/24/32 or float32 input,
stereo float32 output with non-finite samples written as 0.
"""

from __future__ import annotations

import struct

import numpy as np

RATE = 44_100


def sine_mix(seconds: float, seed: int, channels: int = 2, partials: int = 6,
             f_lo: float = 80.0, f_hi: float = 4000.0, a_lo: float = 0.02, a_hi: float = 0.1,
             noise: float = 0.01, rate: int = RATE) -> np.ndarray:
    """Planar [channels][samples] float32 mix: per channel `partials` sines with
    f ~ U(f_lo, f_hi) Hz, amplitude ~ U(a_lo, a_hi), phase ~ U(0, 2*pi), plus
    white noise N(0, noise^2).  Drawn from numpy's default_rng(seed)."""
    n = max(1, int(round(seconds * rate)))
    rng = np.random.default_rng(seed)
    t = np.arange(n, dtype=np.float64) / rate
    out = np.empty((channels, n), np.float32)
    for c in range(channels):
        f = rng.uniform(f_lo, f_hi, partials)
        a = rng.uniform(a_lo, a_hi, partials)
        ph = rng.uniform(0.0, 2.0 * np.pi, partials)
        x = (a[:, None] * np.sin(2.0 * np.pi * f[:, None] * t[None, :] + ph[:, None])).sum(0)
        x += rng.normal(0.0, noise, n)
        out[c] = x.astype(np.float32)
    return out


def write_wav_float(path, planar: np.ndarray, rate: int = RATE) -> None:
    """Stereo/mono IEEE-float32 WAV from planar [C][N]."""
    c, n = planar.shape
    inter = np.ascontiguousarray(planar.T.astype(np.float32))
    data = inter.tobytes()
    hdr = b"RIFF" + struct.pack("<I", 36 + len(data)) + b"WAVEfmt "
    hdr += struct.pack("<IHHIIHH", 16, 3, c, rate, rate * c * 4, c * 4, 32)
    hdr += b"data" + struct.pack("<I", len(data))
    with open(path, "wb") as f:
        f.write(hdr + data)


def read_wav_float(path) -> tuple[np.ndarray, int]:
    """Planar [C][N] float32 from an IEEE-float32 WAV (the host's output)."""
    raw = open(path, "rb").read()
    if raw[:4] != b"RIFF" or raw[8:12] != b"WAVE":
        raise ValueError("not a RIFF/WAVE file")
    off, fmt, ch, rate, bits, payload = 12, 0, 0, 0, 0, None
    while off + 8 <= len(raw):
        cid = raw[off:off + 4]
        (size,) = struct.unpack_from("<I", raw, off + 4)
        body = off + 8
        if cid == b"fmt " and size >= 16:
            fmt, ch, rate = struct.unpack_from("<HHI", raw, body)
            (bits,) = struct.unpack_from("<H", raw, body + 14)
        elif cid == b"data":
            payload = raw[body:body + size]
        off = body + size + (size & 1)
    if fmt != 3 or bits != 32 or payload is None:
        raise ValueError("expected float32 WAV")
    x = np.frombuffer(payload, np.float32).reshape(-1, ch).T.copy()
    return x, rate


def compare(reference: np.ndarray, test: np.ndarray) -> dict:
    """max |delta| and SNR (dB) of `test` against `reference`."""
    r = np.asarray(reference, np.float64).ravel()
    t = np.asarray(test, np.float64).ravel()
    if r.shape != t.shape:
        raise ValueError(f"shape mismatch {r.shape} vs {t.shape}")
    err = t - r
    max_abs = float(np.max(np.abs(err))) if err.size else 0.0
    p_sig = float(np.sum(r * r))
    p_err = float(np.sum(err * err))
    if p_err == 0.0:
        snr = float("inf")
    elif p_sig == 0.0:
        snr = float("-inf")
    else:
        snr = 10.0 * np.log10(p_sig / p_err)
    return {"max_abs": max_abs, "snr_db": snr, "ref_rms": float(np.sqrt(p_sig / max(1, r.size)))}
