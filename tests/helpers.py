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
