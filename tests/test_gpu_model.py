"""Device pipeline (vocalarc_hip.h model entry points) vs the oracle.

Stage tests compare one stage at a time on identical inputs; the forward and
chunked tests compare whole waveforms at the fp32 parity bar: per-sample
max |delta| <= 1e-4 and SNR >= 80 dB.
"""

import numpy as np
import pytest

from helpers import assert_close, empty_dev, from_dev, gpu_available, snr_db, to_dev

pytestmark = pytest.mark.gpu

if gpu_available():
    import oracle as O
    from vocalarc_hip import audio, native, pack
    from vocalarc_hip.dims import CONFIG_DIMS, REFERENCE_DIMS


@pytest.fixture(scope="module")
def ctx():
    if not gpu_available():
        pytest.skip("no GPU")
    c = native.Context()
    yield c
    c.close()


@pytest.fixture(scope="module")
def cfg2():
    """Config shape (dim 384, 62 bands, hop 441, GELU-GLU) at depth 2."""
    d = CONFIG_DIMS.with_depth(2)
    return d, pack.synthetic_pack(d, 77)


@pytest.fixture(scope="module")
def cfg2_models(ctx, cfg2):
    d, blob = cfg2
    return O.Model(d, blob), native.Model(ctx, d, blob)


@pytest.fixture(scope="module")
def ref_models(ctx, ref_pack):
    return O.Model(REFERENCE_DIMS, ref_pack), native.Model(ctx, REFERENCE_DIMS, ref_pack)


@pytest.mark.parametrize("axis,S,L", [(0, 4, 62), (1, 3, 130), (0, 2, 801)])
def test_transformer_block_config(cfg2_models, rng, axis, S, L):
    om, dm = cfg2_models
    x = rng.standard_normal((S, L, om.d.dim), dtype=np.float32)
    ref = om.transformer(1, axis, x, S, L)
    dx = to_dev(x)
    dm.transformer(1, axis, dx, S, L)
    out = from_dev(dx)
    assert_close(ref, out, rtol=1e-4, atol=1e-4, min_snr=100, what="transformer (config)")


@pytest.mark.parametrize("axis,S,L", [(0, 4, 62), (1, 3, 801), (1, 2, 97)])
def test_transformer_block_kv_prescale_bit_identical(cfg2_models, rng, monkeypatch, axis, S, L):
    """The fused block's QKV GEMM writes k and v times the attention's piece
    scales (2^ek, 2^ev: one ldexp exponent per 32-column tile) and the
    attention stages them unscaled; VOCALARC_KV_PRESCALE=0 keeps the
    unscaled projection and the scaling multiplies in the attention.  Both
    must give the same bits (powers of two commute with the rotation and the
    splits), on both axes and on a ragged length.  The band axis runs its
    projection and attention as the two kernels here (VOCALARC_BAND_FUSED=0:
    the fused kernel always scales k and v in its epilogue)."""
    om, dm = cfg2_models
    x = rng.standard_normal((S, L, om.d.dim), dtype=np.float32)
    monkeypatch.setenv("VOCALARC_BAND_FUSED", "0")
    outs = []
    for env in (None, "0"):
        if env is None:
            monkeypatch.delenv("VOCALARC_KV_PRESCALE", raising=False)
        else:
            monkeypatch.setenv("VOCALARC_KV_PRESCALE", env)
        dx = to_dev(x)
        dm.transformer(1, axis, dx, S, L)
        outs.append(from_dev(dx))
    monkeypatch.delenv("VOCALARC_KV_PRESCALE", raising=False)
    monkeypatch.delenv("VOCALARC_BAND_FUSED", raising=False)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


@pytest.mark.parametrize("S,L", [(4, 62), (23, 62), (5, 64), (7, 17), (3, 1)])
def test_band_attention_fused(cfg2_models, rng, monkeypatch, S, L):
    """The band axis's pre-norm projection and attention in one kernel
    (sequences of L <= 64 consecutive rows; q, k, v and the gate logits stay
    on chip), against the oracle and against the two kernels it replaces
    (VOCALARC_BAND_FUSED=0).  q, k and v are formed by the same expressions
    as the QKV GEMM's; the gate logit is an fp32 dot product instead of the
    split GEMM's column, so the two paths agree to a few fp32 roundings of the
    gate, not bit for bit.  Odd S leaves a tile with one sequence, L = 64
    fills a tile's 64 positions, L = 1 is a single key."""
    om, dm = cfg2_models
    x = rng.standard_normal((S, L, om.d.dim), dtype=np.float32)
    outs = []
    for env in (None, "0"):
        if env is None:
            monkeypatch.delenv("VOCALARC_BAND_FUSED", raising=False)
        else:
            monkeypatch.setenv("VOCALARC_BAND_FUSED", env)
        dx = to_dev(x)
        dm.transformer(1, 1, dx, S, L)
        outs.append(from_dev(dx))
    monkeypatch.delenv("VOCALARC_BAND_FUSED", raising=False)
    ref = om.transformer(1, 1, x, S, L)
    assert_close(ref, outs[0], rtol=1e-4, atol=1e-4, min_snr=100, what="fused band attention (oracle)")
    scale = float(np.max(np.abs(outs[1])))
    assert float(np.max(np.abs(outs[0] - outs[1]))) <= 1e-5 * scale
    assert snr_db(outs[1], outs[0]) >= 120.0


@pytest.mark.parametrize("windows", [1, 3])
def test_kv_pieces_bit_identical(cfg2_models, monkeypatch, windows):
    """On the pipeline's time axis (L > 64, [chunk][frame][band] rows) the
    fused QKV GEMM writes k, rotated, and v as the attention's fp16 pieces
    and the attention copies them into LDS by DMA, reading V^T through the
    transpose load; VOCALARC_KV_PIECES=0 keeps the fp32 projection and the
    attention's own rotation and splits.  Both must give the same bits: one
    2 s window (T = 201: ragged query and key blocks) and three 2 s windows
    in one pass (M = 37386 rows: a ragged last row tile, waves whose 32 rows
    straddle two frames, and frames that wrap to the next window)."""
    om, dm = cfg2_models
    chunk, step = 88200, 66150
    x = audio.sine_mix(2.0 if windows == 1 else 5.0, 15)
    length = x.shape[1]
    assert O.chunk_count(length, chunk, step) == windows
    outs = []
    for env in (None, "0"):
        if env is None:
            monkeypatch.delenv("VOCALARC_KV_PIECES", raising=False)
        else:
            monkeypatch.setenv("VOCALARC_KV_PIECES", env)
        dv = empty_dev(x.shape)
        if windows == 1:
            dm.forward(to_dev(x), length, dv)
        else:
            dm.separate(to_dev(x), length, chunk, step, windows, dv)
        outs.append(from_dev(dv))
    monkeypatch.delenv("VOCALARC_KV_PIECES", raising=False)
    assert np.all(np.isfinite(outs[0]))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


@pytest.mark.parametrize("axis,S,L", [(0, 90, 23), (1, 23, 90)])
def test_transformer_block_reference_shape(ref_models, rng, axis, S, L):
    om, dm = ref_models
    x = rng.standard_normal((S, L, om.d.dim), dtype=np.float32)
    ref = om.transformer(5, axis, x, S, L)
    dx = to_dev(x)
    dm.transformer(5, axis, dx, S, L)
    assert_close(ref, from_dev(dx), rtol=1e-4, atol=1e-4, min_snr=100, what="transformer (reference)")


def _to_layout(spec: np.ndarray, layout: int) -> np.ndarray:
    """[F][C][T][2] -> the device layout (frame-major: [C][T][F][2])."""
    return spec if layout == native.SPEC_REFERENCE else np.ascontiguousarray(spec.transpose(1, 2, 0, 3))


def _from_layout(spec: np.ndarray, layout: int) -> np.ndarray:
    return spec if layout == native.SPEC_REFERENCE else np.ascontiguousarray(spec.transpose(2, 0, 1, 3))


LAYOUTS = [0, 1]  # SPEC_REFERENCE, SPEC_FRAME_MAJOR


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("which", ["config", "reference"])
def test_stft_istft(ctx, cfg2_models, ref_models, which, layout):
    om, dm = cfg2_models if which == "config" else ref_models
    d = om.d
    x = audio.sine_mix(0.5, 3)
    length = x.shape[1]
    T = d.frames(length)
    src = O.stft(d, x)
    dsrc = empty_dev(_to_layout(src, layout).shape)
    dm.stft(to_dev(x), length, dsrc, layout)
    gsrc = _from_layout(from_dev(dsrc), layout)
    assert_close(src, gsrc, rtol=1e-6, atol=2e-6, min_snr=120, what="stft")
    rng = np.random.default_rng(5)
    mask = rng.standard_normal(src.shape).astype(np.float32)
    ref = O.istft(d, src, mask, length)
    dout = empty_dev((d.channels, length))
    dm.istft(to_dev(_to_layout(src, layout)), to_dev(_to_layout(mask, layout)), length, dout, layout)
    assert_close(ref, from_dev(dout), rtol=1e-5, atol=1e-6, min_snr=120, what="istft")
    assert T == src.shape[2]


def test_istft_perfect_reconstruction(ctx, cfg2_models):
    """A unit mask reproduces the input (closed form: Hann OLA normalised by
    the summed squared window)."""
    om, dm = cfg2_models
    d = om.d
    x = audio.sine_mix(0.4, 9)
    length = x.shape[1]
    dsrc = empty_dev((d.freq_bins, d.channels, d.frames(length), 2))
    dm.stft(to_dev(x), length, dsrc)
    ones = np.zeros((d.freq_bins, d.channels, d.frames(length), 2), np.float32)
    ones[..., 0] = 1.0
    dout = empty_dev((d.channels, length))
    dm.istft(dsrc, to_dev(ones), length, dout)
    assert_close(x, from_dev(dout), rtol=0, atol=2e-6, what="istft(stft(x))")


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("which", ["config", "reference"])
def test_band_split_and_mask(ctx, cfg2_models, ref_models, which, rng, layout):
    om, dm = cfg2_models if which == "config" else ref_models
    d = om.d
    x = audio.sine_mix(0.3, 4)
    src = O.stft(d, x)
    T = src.shape[2]
    ref = om.band_split(src)
    dout = empty_dev(ref.shape)
    dm.band_split(to_dev(_to_layout(src, layout)), T, dout, layout)
    assert_close(ref, from_dev(dout), rtol=1e-4, atol=2e-5, min_snr=110, what="band split")
    feats = rng.standard_normal((T, d.bands, d.dim), dtype=np.float32)
    mref = om.mask_estimate(feats)
    dmask = empty_dev(_to_layout(mref, layout).shape)
    dm.mask_estimate(to_dev(feats), T, dmask, layout)
    assert_close(mref, _from_layout(from_dev(dmask), layout), rtol=1e-4, atol=1e-5, min_snr=110,
                 what="mask estimator")


def test_forward_config_shape(cfg2_models):
    om, dm = cfg2_models
    x = audio.sine_mix(0.5, 11)
    ref = om.forward(x)
    dv, di = empty_dev(x.shape), empty_dev(x.shape)
    dm.forward(to_dev(x), x.shape[1], dv, di)
    out = from_dev(dv)
    err = float(np.max(np.abs(out.astype(np.float64) - ref)))
    print(f"forward (dim 384, depth 2, 0.5 s): max|d| {err:.3e}, SNR {snr_db(ref, out):.1f} dB")
    assert err <= 1e-4, err
    assert snr_db(ref, out) >= 80
    # instrumental = mix - vocals, computed on the device from the same vocals
    assert np.array_equal(from_dev(di), x - out)


def test_forward_band_unfused(cfg2_models, monkeypatch):
    """The whole forward with the band axis on the two separate kernels
    (VOCALARC_BAND_FUSED=0: the QKV GEMM, then attention_short_h2_kernel)
    against the oracle and against the default, fused path: the path the
    pipeline no longer takes by default stays at the parity bar."""
    om, dm = cfg2_models
    x = audio.sine_mix(0.5, 13)
    ref = om.forward(x)
    outs = []
    for env in ("0", None):
        if env is None:
            monkeypatch.delenv("VOCALARC_BAND_FUSED", raising=False)
        else:
            monkeypatch.setenv("VOCALARC_BAND_FUSED", env)
        dv = empty_dev(x.shape)
        dm.forward(to_dev(x), x.shape[1], dv)
        outs.append(from_dev(dv))
    monkeypatch.delenv("VOCALARC_BAND_FUSED", raising=False)
    for out in outs:
        assert float(np.max(np.abs(out.astype(np.float64) - ref))) <= 1e-4
        assert snr_db(ref, out) >= 80
    assert snr_db(outs[0], outs[1]) >= 110


def test_forward_reference_shape(ref_models):
    om, dm = ref_models
    x = audio.sine_mix(0.2, 12)
    ref = om.forward(x)
    dv = empty_dev(x.shape)
    dm.forward(to_dev(x), x.shape[1], dv)
    out = from_dev(dv)
    err = float(np.max(np.abs(out.astype(np.float64) - ref)))
    print(f"forward (reference shape, depth 16, 0.2 s): max|d| {err:.3e}, SNR {snr_db(ref, out):.1f} dB")
    assert err <= 1e-4, err
    assert snr_db(ref, out) >= 80


def test_chunked_separation(ctx):
    d = CONFIG_DIMS.with_depth(1)
    blob = pack.synthetic_pack(d, 91)
    om, dm = O.Model(d, blob), native.Model(ctx, d, blob)
    x = audio.sine_mix(1.0, 13)
    chunk, step = 13230, 8820  # 0.3 s windows every 0.2 s -> 5 chunks
    ref = om.separate_chunked(x, chunk, step)
    dv, di = empty_dev(x.shape), empty_dev(x.shape)
    dm.separate(to_dev(x), x.shape[1], chunk, step, 2, dv, di)
    out = from_dev(dv)
    assert O.chunk_count(x.shape[1], chunk, step) == 5
    assert np.array_equal(from_dev(di), x - out)
    err = float(np.max(np.abs(out.astype(np.float64) - ref)))
    print(f"chunked separation (5 windows, batch 2): max|d| {err:.3e}, SNR {snr_db(ref, out):.1f} dB")
    assert err <= 1e-4, err
    assert snr_db(ref, out) >= 80
