"""Shared test helpers: device transfer and comparison."""

from __future__ import annotations

import numpy as np


def to_dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def empty_dev(shape, dtype=None):
    import torch
    return torch.empty(shape, dtype=dtype or torch.float32, device="cuda:0")


def from_dev(t) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def snr_db(ref: np.ndarray, test: np.ndarray) -> float:
    r = np.asarray(ref, np.float64).ravel()
    e = np.asarray(test, np.float64).ravel() - r
    pe = float(np.sum(e * e))
    if pe == 0.0:
        return float("inf")
    return 10.0 * np.log10(float(np.sum(r * r)) / pe)


def assert_close(ref, test, rtol: float, atol: float, min_snr: float | None = None, what: str = ""):
    ref = np.asarray(ref)
    test = np.asarray(test)
    assert ref.shape == test.shape, f"{what}: shape {test.shape} != {ref.shape}"
    assert np.all(np.isfinite(test)), f"{what}: non-finite output"
    err = np.abs(test.astype(np.float64) - ref.astype(np.float64))
    lim = atol + rtol * np.abs(ref.astype(np.float64))
    bad = err > lim
    if bad.any():
        i = np.unravel_index(np.argmax(err - lim), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {err.size} elements out of tolerance; worst at {i}: "
                             f"ref {ref[i]!r} test {test[i]!r} (max |d| {err.max():.3e})")
    if min_snr is not None:
        s = snr_db(ref, test)
        assert s >= min_snr, f"{what}: SNR {s:.1f} dB < {min_snr} dB"


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # noqa: BLE001
        return False


def fade64(chunk: int, step: int, index: int, count: int) -> np.ndarray:
    """Closed form of the chunked separation's linear cross-fade over the
    overlap O = chunk - step: every window but the first rises as
    (i + 1/2)/O over its first O samples, every window but the last falls as
    (chunk - i - 1/2)/O over its last O samples, 1 elsewhere (float64)."""
    o = chunk - step
    i = np.arange(chunk, dtype=np.float64)
    w = np.ones(chunk)
    if index > 0:
        w[:o] = (i[:o] + 0.5) / o
    if index + 1 < count:
        w[chunk - o:] = (chunk - i[chunk - o:] - 0.5) / o
    return w


def compose_windows(outs, length: int, chunk: int, step: int, weights=None, starts=None) -> np.ndarray:
    """float64 overlap-add of per-window outputs [C][chunk]:
    sum_k w_k * out_k / sum_k w_k over the samples each window covers (the
    part of the last window past `length` is dropped)."""
    count = len(outs)
    weights = weights or [fade64(chunk, step, k, count) for k in range(count)]
    starts = starts or [k * step for k in range(count)]
    num = np.zeros((outs[0].shape[0], length))
    den = np.zeros(length)
    for k in range(count):
        a = starts[k]
        n = min(length, a + chunk) - a
        num[:, a:a + n] += weights[k][:n] * np.asarray(outs[k], np.float64)[:, :n]
        den[a:a + n] += weights[k][:n]
    return num / den
