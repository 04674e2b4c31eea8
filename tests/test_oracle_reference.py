"""Pin the oracle to the reference implementation (CPU only).

* Row kernels vs the reference's own AVX2/FMA kernels (native/native_simd.c,
  compiled from the reference sources into oracle/_ref/libref_simd.so):
  matmul, dot, axpy and scale bit for bit.  RMSNorm within 5e-7 relative: the
  reference build (-ffast-math, native/Makefile:4) turns
  sqrtf(d)/sqrtf(s) into an RSQRTSS estimate plus one Newton step, a
  CPU-vendor-specific approximation; the oracle uses correctly rounded sqrt
  and division.
* End to end vs the reference CPU executable on a seeded pack and input,
  stage by stage through VOCALARC_DEBUG_DUMP.
* The same end-to-end comparison against the committed fixture
  tests/golden/reference_tiny.npz (made by tests/golden/make_golden.py), which
  keeps the oracle pinned where the reference sources are absent.
"""

import ctypes
import tempfile
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from helpers import snr_db
from vocalarc_hip import audio, pack
from vocalarc_hip.dims import REFERENCE_DIMS as RD

GOLDEN = Path(__file__).parent / "golden" / "reference_tiny.npz"
F = ctypes.POINTER(ctypes.c_float)


def _p(a):
    return a.ctypes.data_as(F)


@pytest.fixture(scope="module")
def simd():
    if not O.REF_SIMD.exists():
        pytest.skip("reference kernels not built (make -C oracle ref)")
    return O.RefSimd().L


@pytest.fixture(scope="module")
def lib():
    L = O.lib()
    L.or_rms_norm_row.argtypes = [F, F, F, ctypes.c_int]
    L.or_matmul_row.argtypes = [F, F, F, F, ctypes.c_int, ctypes.c_int]
    L.or_dot.argtypes = [F, F, ctypes.c_int]
    L.or_axpy.argtypes = [F, F, ctypes.c_float, ctypes.c_int]
    L.or_scale.argtypes = [F, ctypes.c_float, ctypes.c_int]
    return L


@pytest.mark.parametrize("in_dim,out", [(256, 1536), (256, 8), (512, 256), (8, 256), (516, 256), (1024, 1032),
                                        (1024, 16), (384, 3072), (1536, 384)])
def test_matmul_row_bit_exact(simd, lib, rng, in_dim, out):
    for _ in range(3):
        x = rng.standard_normal(in_dim).astype(np.float32)
        w = (0.02 * rng.standard_normal(in_dim * out)).astype(np.float32)
        b = rng.standard_normal(out).astype(np.float32)
        y1, y2 = np.empty(out, np.float32), np.empty(out, np.float32)
        simd.vocalarc_matmul_row_avx2(_p(x), _p(w), _p(b), _p(y1), in_dim, out)
        lib.or_matmul_row(_p(x), _p(w), _p(b), _p(y2), in_dim, out)
        assert np.array_equal(y1, y2)


def test_dot_axpy_scale_bit_exact(simd, lib, rng):
    for n in (64, 8, 72):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        assert simd.vocalarc_dot_avx2(_p(a), _p(b), n) == lib.or_dot(_p(a), _p(b), n)
    d1 = rng.standard_normal(64).astype(np.float32)
    d2 = d1.copy()
    s = rng.standard_normal(64).astype(np.float32)
    simd.vocalarc_axpy_avx2(_p(d1), _p(s), ctypes.c_float(0.37))
    lib.or_axpy(_p(d2), _p(s), ctypes.c_float(0.37), 64)
    assert np.array_equal(d1, d2)
    simd.vocalarc_scale_head_avx2(_p(d1), ctypes.c_float(0.91))
    lib.or_scale(_p(d2), ctypes.c_float(0.91), 64)
    assert np.array_equal(d1, d2)


@pytest.mark.parametrize("dim", [8, 16, 48, 96, 192, 256, 384, 512, 516])
def test_rms_norm_row_within_rsqrt_bound(simd, lib, rng, dim):
    """One Newton step on a 12-bit RSQRTSS estimate leaves ~2e-7 relative
    error in the scale; two float multiplies add an ulp each."""
    for _ in range(20):
        x = rng.standard_normal(dim).astype(np.float32) * np.float32(rng.uniform(0.01, 10))
        g = (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
        y1, y2 = np.empty(dim, np.float32), np.empty(dim, np.float32)
        simd.vocalarc_rms_norm_row_avx2(_p(x), _p(g), _p(y1), dim)
        lib.or_rms_norm_row(_p(x), _p(g), _p(y2), dim)
        assert np.all(np.abs(y1.astype(np.float64) - y2) <= 5e-7 * np.abs(y2.astype(np.float64)))


def _stage_checks(stages: dict, mine: dict):
    """Per-stage agreement: the STFT is fp64 internally (bit-level), the
    stages after an RMSNorm carry its few-ulp difference (>= 110 dB)."""
    assert snr_db(stages["source"], mine["source"]) > 250
    for name in ("band", "features1", "features16", "mask", "vocals", "instrumental"):
        s = snr_db(stages[name], mine[name])
        assert s >= 110, (name, s)
    scale = float(np.max(np.abs(stages["vocals"])))
    assert float(np.max(np.abs(stages["vocals"].astype(np.float64) - mine["vocals"]))) <= 1e-5 * scale


def test_oracle_matches_golden_fixture(ref_pack):
    g = np.load(GOLDEN)
    assert int(g["pack_seed"]) == 1234
    x = g["audio"]
    m = O.Model(RD, ref_pack)
    v, dumps = m.forward(x, dumps=True)
    stride = int(g["feature_stride"])
    mine = {"source": dumps["source"].ravel(), "band": dumps["band"].ravel()[::stride],
            "features1": dumps["features1"].ravel()[::stride], "features16": dumps["features_last"].ravel()[::stride],
            "mask": dumps["mask"].ravel(), "vocals": v, "instrumental": x - v}
    _stage_checks({k: g[k] for k in ("source", "band", "features1", "features16", "mask", "vocals", "instrumental")},
                  mine)


def test_oracle_matches_reference_executable(ref_pack):
    if not O.REF_EXE.exists():
        pytest.skip("reference executable not built (make -C oracle ref)")
    x = audio.sine_mix(0.12, 99)
    with tempfile.TemporaryDirectory() as tmp:
        t = Path(tmp)
        pack.write_pack(t / "m.f32", ref_pack)
        audio.write_wav_float(t / "in.wav", x)
        resp = O.run_reference(O.REF_EXE, t / "m.f32", t / "in.wav", t / "v.wav", t / "i.wav", threads=8,
                               dump_prefix=str(t / "d"))
        sep = [r for r in resp if r.get("type") == "separated"][0]
        assert sep["frames"] == RD.frames(x.shape[1])
        ref = {n: np.fromfile(t / f"d-{n}.f32", np.float32)
               for n in ("source", "band", "features1", "features16", "mask")}
        ref["vocals"] = audio.read_wav_float(t / "v.wav")[0]
        ref["instrumental"] = audio.read_wav_float(t / "i.wav")[0]
    m = O.Model(RD, ref_pack)
    v, dumps = m.forward(x, dumps=True)
    mine = {"source": dumps["source"].ravel(), "band": dumps["band"].ravel(), "features1": dumps["features1"].ravel(),
            "features16": dumps["features_last"].ravel(), "mask": dumps["mask"].ravel(), "vocals": v,
            "instrumental": x - v}
    _stage_checks(ref, mine)


def test_reference_grouping_is_bit_invariant(ref_pack):
    """The host's sequence grouping (timeBandGroup/frequencyFrameGroup) does
    not change a bit of the output, so the provider's full batches and the
    host's bounded groups are comparable (native/vocalarc_separation.c:1396-1420)."""
    if not O.REF_EXE.exists():
        pytest.skip("reference executable not built")
    x = audio.sine_mix(0.06, 5)
    outs = []
    with tempfile.TemporaryDirectory() as tmp:
        t = Path(tmp)
        pack.write_pack(t / "m.f32", ref_pack)
        audio.write_wav_float(t / "in.wav", x)
        for groups in ((90, 6), (7, 3)):
            O.run_reference(O.REF_EXE, t / "m.f32", t / "in.wav", t / "v.wav", threads=4, groups=groups)
            outs.append(audio.read_wav_float(t / "v.wav")[0])
    assert np.array_equal(outs[0], outs[1])
