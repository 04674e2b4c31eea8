"""Every benchmark configuration at its own size, on the device, against the oracle.

C1  isolated kernels: the row softmax over [62*8*801, 801] scores (the other
    C1 kernels run at their full sizes in test_gpu_kernels.py);
C2  one axial layer on [801 frames, 62 bands, 384]: the time transformer
    (62 sequences of 801) and the band transformer (801 sequences of 62);
C3  the DSP front and back end on 60 s of audio (hop 441, T = 6001):
    STFT, masked iSTFT, band split and mask estimator;
C4  the depth-12 model: one whole 8 s window (fp32 and the bf16 variant),
    a 3-window chunked separation (8 s windows, 6 s step, zero-padded tail),
    and the benchmark's own launch shape -- a 50 s mix cut into 8 windows
    that go through the device in ONE pass (time axis 496 sequences of 801,
    band axis 6408 sequences of 62, 397,296 tokens per GEMM), one window
    of digital silence among them -- each against the oracle's window
    forwards composed with the closed-form cross-fade (the composition is
    pinned to the oracle's chunked separation on the CPU,
    test_oracle_math.py).
C0  (the 10 s host path) runs in test_gpu_abi.py.

Bars: fp32 waveforms per-sample max |delta| <= 1e-4 and SNR >= 80 dB; the
bf16 variant SNR >= 40 dB; stages as in the smaller-size tests.
"""

import numpy as np
import pytest

from helpers import assert_close, compose_windows, empty_dev, from_dev, gpu_available, snr_db, to_dev

pytestmark = pytest.mark.gpu

if gpu_available():
    import oracle as O
    from vocalarc_hip import audio, native, pack
    from vocalarc_hip.dims import CONFIG_DIMS

RATE = 44100


@pytest.fixture(scope="module")
def ctx():
    if not gpu_available():
        pytest.skip("no GPU")
    c = native.Context()
    yield c
    c.close()


def _close_chunked(ref, out, rtol, atol, what, rows=1 << 16):
    """assert_close over row blocks (keeps float64 temporaries small)."""
    ref2 = ref.reshape(-1, ref.shape[-1])
    out2 = out.reshape(-1, out.shape[-1])
    for r0 in range(0, ref2.shape[0], rows):
        assert_close(ref2[r0:r0 + rows], out2[r0:r0 + rows], rtol=rtol, atol=atol, what=f"{what} rows {r0}+")


def _wave_bar(ref, out, what, max_abs=1e-4, min_snr=80.0):
    assert np.all(np.isfinite(out)), what
    err = float(np.max(np.abs(out.astype(np.float64) - ref)))
    snr = snr_db(ref, out)
    print(f"{what}: max|d| {err:.3e}, SNR {snr:.1f} dB")
    assert err <= max_abs, (what, err)
    assert snr >= min_snr, (what, snr)


# ------------------------------------------------------------------ C1

def test_c1_softmax_full(ctx):
    """Row softmax over [62*8, 801, 801] = 318.2 M scores, inputs N(0, 1)."""
    rows, length = 62 * 8 * 801, 801
    x = np.random.default_rng(101).standard_normal((rows, length), dtype=np.float32)
    dx = to_dev(x)
    dy = empty_dev((rows, length))
    ctx.softmax_rows(dx, dy, rows, length)
    ctx.sync()
    del dx
    out = from_dev(dy)
    del dy
    ref = O.softmax_rows(x)
    del x
    _close_chunked(ref, out, rtol=1e-5, atol=1e-9, what="softmax [496*801, 801]")
    sums = out.astype(np.float64).sum(-1)
    assert np.allclose(sums, 1.0, atol=1e-5)


# ------------------------------------------------------------------ C2

@pytest.fixture(scope="module")
def layer_setup(ctx):
    d = CONFIG_DIMS.with_depth(1)
    blob = pack.synthetic_pack(d, 202)
    x = np.random.default_rng(203).standard_normal((801, d.bands, d.dim), dtype=np.float32)  # [frames][bands][dim]
    return d, O.Model(d, blob), native.Model(ctx, d, blob), x


def test_c2_full_layer_both_axes(layer_setup):
    d, om, dm, x = layer_setup
    T, B = x.shape[0], x.shape[1]
    # time transformer: 62 sequences (bands) of 801 frames
    xt = np.ascontiguousarray(x.transpose(1, 0, 2))
    ref_t = om.transformer(0, 0, xt, B, T)
    dxt = to_dev(xt)
    dm.transformer(0, 0, dxt, B, T)
    out_t = from_dev(dxt)
    assert_close(ref_t, out_t, rtol=1e-4, atol=1e-4, min_snr=100, what="C2 time transformer [62, 801, 384]")
    # band transformer on the oracle's time output: 801 sequences (frames) of 62 bands
    xb = np.ascontiguousarray(ref_t.transpose(1, 0, 2))
    ref_b = om.transformer(0, 1, xb, T, B)
    dxb = to_dev(xb)
    dm.transformer(0, 1, dxb, T, B)
    assert_close(ref_b, from_dev(dxb), rtol=1e-4, atol=1e-4, min_snr=100, what="C2 band transformer [801, 62, 384]")
    # the whole layer chained on the device
    dxb2 = to_dev(np.ascontiguousarray(out_t.transpose(1, 0, 2)))
    dm.transformer(0, 1, dxb2, T, B)
    out = from_dev(dxb2)
    print(f"C2 layer chained on the device: SNR {snr_db(ref_b, out):.1f} dB")
    assert_close(ref_b, out, rtol=1e-4, atol=1e-4, min_snr=100, what="C2 layer (time then band)")


# ------------------------------------------------------------------ C3

@pytest.fixture(scope="module")
def dsp_setup(ctx):
    d = CONFIG_DIMS.with_depth(1)
    blob = pack.synthetic_pack(d, 303)
    x = audio.sine_mix(60.0, 304)
    return d, O.Model(d, blob), native.Model(ctx, d, blob), x


@pytest.mark.parametrize("layout", [0, 1])  # SPEC_REFERENCE, SPEC_FRAME_MAJOR
def test_c3_stft_istft_60s(dsp_setup, layout):
    d, om, dm, x = dsp_setup
    length = x.shape[1]
    T = d.frames(length)
    assert T == 6001
    src = O.stft(d, x)

    def to_layout(a):
        return a if layout == 0 else np.ascontiguousarray(a.transpose(1, 2, 0, 3))

    def from_layout(a):
        return a if layout == 0 else np.ascontiguousarray(a.transpose(2, 0, 1, 3))

    dsrc = empty_dev(to_layout(src).shape)
    dm.stft(to_dev(x), length, dsrc, layout)
    assert_close(src, from_layout(from_dev(dsrc)), rtol=1e-6, atol=2e-6, min_snr=120, what="C3 STFT 60 s")
    mask = np.random.default_rng(305).standard_normal(src.shape).astype(np.float32)
    ref = O.istft(d, src, mask, length)
    dout = empty_dev((d.channels, length))
    dm.istft(to_dev(to_layout(src)), to_dev(to_layout(mask)), length, dout, layout)
    assert_close(ref, from_dev(dout), rtol=1e-5, atol=1e-6, min_snr=120, what="C3 masked iSTFT 60 s")


def test_c3_band_split_and_mask_60s(dsp_setup):
    d, om, dm, x = dsp_setup
    src = O.stft(d, x)
    T = src.shape[2]
    ref = om.band_split(src)
    dout = empty_dev(ref.shape)
    dm.band_split(to_dev(src), T, dout)
    assert_close(ref, from_dev(dout), rtol=1e-4, atol=2e-5, min_snr=110, what="C3 band split T=6001")
    feats = np.random.default_rng(306).standard_normal((T, d.bands, d.dim), dtype=np.float32)
    mref = om.mask_estimate(feats)
    dmask = empty_dev(mref.shape)
    dm.mask_estimate(to_dev(feats), T, dmask)
    assert_close(mref, from_dev(dmask), rtol=1e-4, atol=1e-5, min_snr=110, what="C3 mask estimator T=6001")


# ------------------------------------------------------------------ C4

CHUNK, STEP = 8 * RATE, 6 * RATE


@pytest.fixture(scope="module")
def c4(ctx):
    """Depth-12 model at the configuration shape; a 19 s mix cut into 3
    windows of 8 s every 6 s (the last zero-padded by 1 s); the oracle's
    forward of each window."""
    d = CONFIG_DIMS
    assert d.depth == 12
    blob = pack.synthetic_pack(d, 404)
    x = audio.sine_mix(19.0, 405)
    length = x.shape[1]
    count = O.chunk_count(length, CHUNK, STEP)
    assert count == 3 and 2 * STEP + CHUNK > length
    om = O.Model(d, blob)
    outs = []
    for k in range(count):
        win = np.zeros((d.channels, CHUNK), np.float32)
        seg = x[:, k * STEP:min(length, k * STEP + CHUNK)]
        win[:, :seg.shape[1]] = seg
        outs.append(om.forward(win))
    dm = native.Model(ctx, d, blob)
    yield d, dm, x, outs
    dm.set_precision(native.PRECISION_FP32)


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_c4_one_window_depth12(c4, precision):
    d, dm, x, outs = c4
    dm.set_precision(native.PRECISION_FP32 if precision == "fp32" else native.PRECISION_BF16)
    w = np.ascontiguousarray(x[:, :CHUNK])
    dv = empty_dev(w.shape)
    dm.forward(to_dev(w), CHUNK, dv)
    out = from_dev(dv)
    dm.set_precision(native.PRECISION_FP32)
    if precision == "fp32":
        _wave_bar(outs[0], out, "C4 one 8 s window, depth 12, fp32")
    else:
        _wave_bar(outs[0], out, "C4 one 8 s window, depth 12, bf16 variant", max_abs=np.inf, min_snr=40.0)


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_c4_chunked_three_windows_depth12(c4, precision):
    d, dm, x, outs = c4
    length = x.shape[1]
    ref = compose_windows(outs, length, CHUNK, STEP)
    dm.set_precision(native.PRECISION_FP32 if precision == "fp32" else native.PRECISION_BF16)
    dx = to_dev(x)
    dv, di = empty_dev(x.shape), empty_dev(x.shape)
    dm.separate(dx, length, CHUNK, STEP, 8, dv, di)
    out = from_dev(dv)
    dm.set_precision(native.PRECISION_FP32)
    assert np.array_equal(from_dev(di), x - out)
    if precision == "fp32":
        _wave_bar(ref, out, "C4 chunked 3 windows, depth 12, fp32")
    else:
        _wave_bar(ref, out, "C4 chunked 3 windows, depth 12, bf16 variant", max_abs=np.inf, min_snr=40.0)


@pytest.fixture(scope="module")
def c4_pass(ctx):
    """The benchmark's launch shape: a 50 s mix = 8 windows of 8 s every 6 s
    (7 * 6 + 8 = 50, no padding), all 8 in one device pass; samples 18-26 s
    are digital silence, so window 3 is all zeros (its band inputs take the
    RMSNorm's epsilon path, native/vocalarc_separation.c:419-424, and its
    features are the band-split biases alone) and windows 2 and 4 are
    partly silent.  The oracle's forward of each window (depth 12)."""
    d = CONFIG_DIMS
    blob = pack.synthetic_pack(d, 406)
    x = audio.sine_mix(50.0, 407)
    x[:, 18 * RATE:26 * RATE] = 0.0
    length = x.shape[1]
    count = O.chunk_count(length, CHUNK, STEP)
    assert count == 8 and (count - 1) * STEP + CHUNK == length
    om = O.Model(d, blob)
    outs = [om.forward(np.ascontiguousarray(x[:, k * STEP:k * STEP + CHUNK])) for k in range(count)]
    assert not np.any(x[:, 3 * STEP:3 * STEP + CHUNK]) and np.all(np.isfinite(outs[3]))
    dm = native.Model(ctx, d, blob)
    yield d, dm, x, outs
    dm.set_precision(native.PRECISION_FP32)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_c4_eight_windows_one_pass_depth12(c4_pass, precision):
    d, dm, x, outs = c4_pass
    length = x.shape[1]
    ref = compose_windows(outs, length, CHUNK, STEP)
    dm.set_precision(native.PRECISION_FP32 if precision == "fp32" else native.PRECISION_BF16)
    dx = to_dev(x)
    dv, di = empty_dev(x.shape), empty_dev(x.shape)
    dm.separate(dx, length, CHUNK, STEP, 8, dv, di)
    out = from_dev(dv)
    dm.set_precision(native.PRECISION_FP32)
    assert np.array_equal(from_dev(di), x - out)
    silent = slice(3 * STEP, 3 * STEP + CHUNK)
    if precision == "fp32":
        _wave_bar(ref, out, "C4 8 windows in one pass, depth 12, fp32")
        # the silent window's span: the mix is zero there, so vocals come
        # only from the edge frames of the overlapping windows 2 and 4
        err = float(np.max(np.abs(out[:, silent].astype(np.float64) - ref[:, silent])))
        print(f"silent span: max|ref| {float(np.max(np.abs(ref[:, silent]))):.3e}, max|d| {err:.3e}")
        assert err <= 1e-4
    else:
        _wave_bar(ref, out, "C4 8 windows in one pass, depth 12, bf16 variant", max_abs=np.inf, min_snr=40.0)
