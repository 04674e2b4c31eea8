"""The oracle against what the mathematics fixes (CPU only).

Each check is an independent float64 computation (numpy / math), not a
restatement of the oracle's C: a dropped term, a wrong sign or index, or a
transposed operand in the oracle fails one of these.
"""

import math

import numpy as np
import pytest

import oracle as O
from helpers import compose_windows, fade64, snr_db
from vocalarc_hip import audio, pack
from vocalarc_hip.dims import BAND_WIDTHS_62, CONFIG_DIMS, REFERENCE_BAND_WIDTHS, REFERENCE_DIMS, ModelDims


def test_fast_exp_accuracy():
    """Range reduction r = x - n*ln2 is evaluated in float, so the error grows
    with |x| (the float product n*ln2 carries half an ulp of ~|x|)."""
    xs = np.linspace(-85.0, 85.0, 20001)
    for x in xs[::7]:
        ref = math.exp(float(np.float32(x)))
        assert abs(O.fast_exp(float(x)) - ref) <= (2e-7 + 6e-8 * abs(x)) * ref
    assert O.fast_exp(-100.0) == 0.0
    assert O.fast_exp(0.0) == 1.0


def test_rms_norm_formula(rng):
    x = rng.standard_normal((50, 384)).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(384)).astype(np.float32)
    x64 = x.astype(np.float64)
    ref = x64 * np.sqrt(384.0) / np.sqrt((x64 ** 2).sum(1, keepdims=True) + 1e-12) * g
    assert np.allclose(O.rms_norm(x, g), ref, rtol=1e-6, atol=1e-7)
    # zero row: eps keeps it finite and zero
    z = O.rms_norm(np.zeros((1, 8), np.float32), np.ones(8, np.float32))
    assert np.all(z == 0)


@pytest.mark.parametrize("in_dim,out", [(256, 1536), (24, 8), (516, 256), (100, 37 * 8)])
def test_matmul_packed_layout(rng, in_dim, out):
    x = rng.standard_normal((9, in_dim)).astype(np.float32)
    w = rng.standard_normal((out, in_dim)).astype(np.float32)
    b = rng.standard_normal(out).astype(np.float32)
    packed = pack.pack_matrix(w)
    assert np.array_equal(pack.unpack_matrix(packed, out, in_dim), w)
    ref = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert np.allclose(O.matmul(x, packed, out, b), ref, rtol=1e-5, atol=1e-4)


def test_pack_layout_tile_order():
    """Element (o, i) of a packed matrix: full tiles [o/32][i][o%32], then the
    tail [i][o-full] (native/vocalarc_separation.c:428-457)."""
    out, inp = 40, 3
    w = np.arange(out * inp, dtype=np.float32).reshape(out, inp)
    p = pack.pack_matrix(w)
    assert p[0 * 32 + 5] == w[5, 0]
    assert p[2 * 32 + 7] == w[7, 2]
    assert p[32 * inp + 1 * 8 + 3] == w[32 + 3, 1]


def test_gelu_and_geglu(rng):
    x = (3 * rng.standard_normal(1000)).astype(np.float32)
    ref = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.astype(np.float64)])
    assert np.allclose(O.gelu(x), ref, rtol=1e-5, atol=1e-6)
    v = rng.standard_normal((5, 8)).astype(np.float32)
    g = rng.standard_normal((5, 8)).astype(np.float32)
    gg = np.array([[0.5 * b * (1 + math.erf(b / math.sqrt(2))) for b in row] for row in g.astype(np.float64)])
    assert np.allclose(O.geglu(np.concatenate([v, g], 1)), v * gg, rtol=1e-5, atol=1e-6)


def test_softmax_rows_closed_form(rng):
    x = (4 * rng.standard_normal((6, 801))).astype(np.float32)
    e = np.exp(x.astype(np.float64) - x.max(1, keepdims=True))
    assert np.allclose(O.softmax_rows(x), e / e.sum(1, keepdims=True), rtol=1e-5, atol=1e-9)


def test_rope_table_and_rotation(rng):
    c, s = O.rope_table(801, 64)
    assert np.allclose(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2, 1.0, atol=1e-6)
    assert np.all(c[0] == 1) and np.all(s[0] == 0)
    # theta = p * 10000^(-2k/64): pair 0 rotates by p radians, pair 31 slowest
    p = 123
    assert abs(math.atan2(s[p, 0], c[p, 0]) - math.remainder(p, 2 * math.pi)) < 1e-4
    f31 = 10000.0 ** (-62 / 64)
    assert abs(c[p, 31] - math.cos(p * f31)) < 1e-6
    # rotating position p of a unit vector along the first axis gives (cos, sin)
    x = np.zeros((1, 801, 64), np.float32)
    x[0, :, 0] = 1.0
    y = O.rope_bhld(x)
    assert np.allclose(y[0, :, 0], c[:, 0]) and np.allclose(y[0, :, 1], s[:, 0])


def _attention64(q, k, v):
    s = q @ k.T / 8.0
    s -= s.max(1, keepdims=True)
    p = np.exp(s)
    return (p / p.sum(1, keepdims=True)) @ v


def test_attention_brute_force(rng):
    d = REFERENCE_DIMS
    S, L, H = 2, 37, d.heads
    qkv = rng.standard_normal((S * L, 3 * H * 64)).astype(np.float32)
    out = O.attention(d, qkv, S, L)
    q64 = qkv.astype(np.float64)
    for s in range(S):
        for h in range(H):
            rows = slice(s * L, (s + 1) * L)
            q = q64[rows, h * 64:(h + 1) * 64]
            k = q64[rows, 512 + h * 64:512 + (h + 1) * 64]
            v = q64[rows, 1024 + h * 64:1024 + (h + 1) * 64]
            assert np.allclose(out[rows, h * 64:(h + 1) * 64], _attention64(q, k, v), rtol=1e-5, atol=2e-6)


def _rms64(x, g):
    return x * np.sqrt(x.shape[-1]) / np.sqrt((x ** 2).sum(-1, keepdims=True) + 1e-12) * g


def _gelu64(x):
    from scipy.special import erf
    return 0.5 * x * (1 + erf(x / np.sqrt(2)))


def _transformer64(d: ModelDims, w, x, S, L):
    """Independent float64 statement of one axial block
    (native/vocalarc_separation.c:836-873) on unpacked weights."""
    H, inner = d.heads, d.inner
    x = x.reshape(S * L, d.dim).astype(np.float64)
    n = _rms64(x, w["gamma"])
    qkv = n @ w["qkv"].T
    pos = np.arange(S * L) % L
    freq = 1.0 / 10000.0 ** (np.arange(32) * 2 / 64)
    ang = pos[:, None] * freq[None, :]
    for which in range(2):
        blk = qkv[:, which * inner:(which + 1) * inner].reshape(-1, H, 32, 2)
        a, b = blk[..., 0].copy(), blk[..., 1].copy()
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        blk[..., 0], blk[..., 1] = a * c - b * s, a * s + b * c
        qkv[:, which * inner:(which + 1) * inner] = blk.reshape(-1, inner)
    att = np.zeros((S * L, inner))
    for sq in range(S):
        r = slice(sq * L, (sq + 1) * L)
        for h in range(H):
            att[r, h * 64:(h + 1) * 64] = _attention64(qkv[r, h * 64:(h + 1) * 64],
                                                        qkv[r, inner + h * 64:inner + (h + 1) * 64],
                                                        qkv[r, 2 * inner + h * 64:2 * inner + (h + 1) * 64])
    if d.gated:
        gates = 1 / (1 + np.exp(-(n @ w["gate_weight"].T + w["gate_bias"])))
        att *= np.repeat(gates, 64, axis=1)
    x = x + att @ w["out_weight"].T
    n = _rms64(x, w["ff_gamma"])
    h1 = n @ w["ff1_weight"].T + w["ff1_bias"]
    if d.ffn_glu:
        h1 = h1[:, :d.ff_dim] * _gelu64(h1[:, d.ff_dim:])
    else:
        h1 = _gelu64(h1)
    x = x + h1 @ w["ff2_weight"].T + w["ff2_bias"]
    return x.reshape(S, L, d.dim)


@pytest.mark.parametrize("glu", [False, True])
def test_transformer_block_float64(glu):
    d = ModelDims(dim=64, depth=1, heads=2, dim_head=64, ff_dim=96 if glu else 128, ffn_glu=glu, gated=True,
                  mask_hidden=64, n_fft=16, hop=4, band_widths=(2, 3, 4), model_frames=0)
    blob = pack.synthetic_pack(d, 3, std=0.1)
    views = pack.tensor_views(d, blob)
    m = O.Model(d, blob)
    w = {}
    for spec in pack.tensor_specs(d):
        if spec.name.startswith("layers.0.1."):
            key = spec.name.split(".")[-1]
            val = views[spec.name].astype(np.float64)
            w[key] = pack.unpack_matrix(views[spec.name], spec.out, spec.inp).astype(np.float64) \
                if spec.kind == "matrix" else val
    rng = np.random.default_rng(1)
    S, L = 3, 11
    x = rng.standard_normal((S, L, d.dim)).astype(np.float32)
    ref = _transformer64(d, w, x, S, L)
    got = m.transformer(0, 1, x, S, L)
    assert snr_db(ref, got) > 110


def test_hann_periodic():
    w = O.hann(2048).astype(np.float64)
    i = np.arange(2048)
    assert np.allclose(w, np.sin(np.pi * i / 2048) ** 2, atol=1e-7)
    # hop 512: the squared window sums to 1.5 everywhere (4x overlap)
    env = sum(np.roll(w ** 2, 512 * k) for k in range(4))
    assert np.allclose(env, 1.5, atol=1e-6)


@pytest.mark.parametrize("dims", [REFERENCE_DIMS, CONFIG_DIMS])
def test_stft_matches_numpy_rfft(dims):
    x = audio.sine_mix(0.2, 8)
    src = O.stft(dims, x)
    N, hop = dims.n_fft, dims.hop
    T = dims.frames(x.shape[1])
    w = np.sin(np.pi * np.arange(N) / N) ** 2
    for c in range(2):
        pad = np.pad(x[c].astype(np.float64), (N // 2, N // 2), mode="reflect")
        for t in (0, 1, T // 2, T - 1):
            spec = np.fft.rfft(pad[t * hop:t * hop + N] * w)
            got = src[:, c, t, 0] + 1j * src[:, c, t, 1]
            assert np.allclose(got, spec, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dims", [REFERENCE_DIMS, CONFIG_DIMS])
def test_istft_perfect_reconstruction(dims):
    x = audio.sine_mix(0.3, 10)
    src = O.stft(dims, x)
    mask = np.zeros_like(src)
    mask[..., 0] = 1
    y = O.istft(dims, src, mask, x.shape[1])
    assert np.max(np.abs(y - x)) < 1e-6
    # a zero mask gives exact silence (the normalised envelope divides zeros)
    mask[..., 0], mask[..., 1] = 0, 0
    assert np.all(O.istft(dims, src, mask, x.shape[1]) == 0)


def _istft64(d, source: np.ndarray, mask: np.ndarray, length: int) -> np.ndarray:
    """float64 statement of the masked inverse STFT: Y = S*M per bin,
    x_t = irfft(Y_t) (the imaginary parts of DC and Nyquist do not reach a
    real signal), windowed by the periodic Hann, overlap-added at t*hop - N/2
    and divided by the summed squared window where that exceeds 1e-12."""
    N, hop = d.n_fft, d.hop
    T = source.shape[2]
    Y = (source[..., 0].astype(np.float64) + 1j * source[..., 1]) * (mask[..., 0] + 1j * mask[..., 1].astype(np.float64))
    w = np.sin(np.pi * np.arange(N) / N) ** 2
    out = np.zeros((d.channels, length))
    env = np.zeros(length)
    for t in range(T):
        frames = np.fft.irfft(Y[:, :, t].T, n=N) * w  # [C][N]
        s0 = t * hop - N // 2
        a, b = max(0, s0), min(length, s0 + N)
        out[:, a:b] += frames[:, a - s0:b - s0]
        env[a:b] += w[a - s0:b - s0] ** 2
    return np.where(env > 1e-12, out / np.where(env > 1e-12, env, 1.0), 0.0)


@pytest.mark.parametrize("dims", [REFERENCE_DIMS, CONFIG_DIMS])
def test_istft_random_complex_mask_matches_numpy(dims, rng):
    """A random complex mask (both parts N(0,1), so the real/imaginary
    cross terms of the complex product all matter) against the float64
    irfft + overlap-add statement."""
    x = audio.sine_mix(0.25, 14)
    src = O.stft(dims, x)
    mask = rng.standard_normal(src.shape).astype(np.float32)
    got = O.istft(dims, src, mask, x.shape[1])
    ref = _istft64(dims, src, mask, x.shape[1])
    scale = float(np.max(np.abs(ref)))
    assert np.max(np.abs(got - ref)) <= 2e-6 * scale
    # a swapped sign in the complex product (S * conj(M)) is far outside that
    conj = mask.copy()
    conj[..., 1] *= -1
    assert np.max(np.abs(_istft64(dims, src, conj, x.shape[1]) - ref)) > 0.1 * scale


def test_band_tables():
    assert len(REFERENCE_BAND_WIDTHS) == 90 and sum(REFERENCE_BAND_WIDTHS) == 1025
    assert len(BAND_WIDTHS_62) == 62 and sum(BAND_WIDTHS_62) == 1025
    assert REFERENCE_DIMS.first_frequencies()[60] == 24 * 2 + 36 * 4
    assert REFERENCE_DIMS.input_dims()[-1] == 129 * 4


def test_band_split_and_mask_float64(rng):
    d = ModelDims(dim=16, depth=0, heads=1, dim_head=64, ff_dim=32, mask_hidden=24, n_fft=16, hop=4,
                  band_widths=(2, 3, 4), model_frames=0)
    blob = pack.synthetic_pack(d, 4, std=0.2)
    v = pack.tensor_views(d, blob)
    m = O.Model(d, blob)
    T = 5
    src = rng.standard_normal((d.freq_bins, 2, T, 2)).astype(np.float32)
    got = m.band_split(src)
    f0 = d.first_frequencies()
    for b, wdt in enumerate(d.band_widths):
        # gather order: frequency, channel, re/im
        inp = src[f0[b]:f0[b] + wdt].transpose(2, 0, 1, 3).reshape(T, -1).astype(np.float64)
        n = _rms64(inp, v[f"bands.{b}.gamma"])
        W = pack.unpack_matrix(v[f"bands.{b}.weight"], d.dim, 4 * wdt).astype(np.float64)
        ref = n @ W.T + v[f"bands.{b}.bias"]
        assert np.allclose(got[b], ref, rtol=1e-5, atol=1e-5)
    feats = rng.standard_normal((T, d.bands, d.dim)).astype(np.float32)
    mask = m.mask_estimate(feats)
    for b, wdt in enumerate(d.band_widths):
        W1 = pack.unpack_matrix(v[f"masks.{b}.first_weight"], d.mask_hidden, d.dim).astype(np.float64)
        W2 = pack.unpack_matrix(v[f"masks.{b}.second_weight"], 8 * wdt, d.mask_hidden).astype(np.float64)
        hdn = np.tanh(feats[:, b].astype(np.float64) @ W1.T + v[f"masks.{b}.first_bias"])
        p = hdn @ W2.T + v[f"masks.{b}.second_bias"]
        glu = p[:, :4 * wdt] / (1 + np.exp(-p[:, 4 * wdt:]))
        ref = glu.reshape(T, wdt, 2, 2).transpose(1, 2, 0, 3)  # [f][c][t][re/im]
        assert np.allclose(mask[f0[b]:f0[b] + wdt], ref, rtol=1e-5, atol=1e-6)


def test_chunk_weights_partition_of_unity():
    chunk, step = 1000, 700
    count = O.chunk_count(5000, chunk, step)
    assert count == 1 + math.ceil((5000 - chunk) / step)
    total = np.zeros(5000 + chunk)
    for k in range(count):
        total[k * step:k * step + chunk] += O.chunk_weights(chunk, step, k, count)
    assert np.allclose(total[:5000], 1.0, atol=1e-6)
    assert O.chunk_count(800, chunk, step) == 1


def _fade64_swapped(chunk: int, step: int, index: int, count: int) -> np.ndarray:
    """A planted mistake: the two fade shapes exchanged (falling over a
    window's first O samples, rising over its last O) -- still a partition
    of unity, so only a composition check can tell it apart."""
    O_ = chunk - step
    i = np.arange(chunk, dtype=np.float64)
    w = np.ones(chunk)
    if index > 0:
        w[:O_] = (O_ - i[:O_] - 0.5) / O_
    if index + 1 < count:
        w[chunk - O_:] = (i[chunk - O_:] - (chunk - O_) + 0.5) / O_
    return w


@pytest.mark.parametrize("chunk,step,index,count", [(1000, 700, 0, 4), (1000, 700, 1, 4), (1000, 700, 3, 4),
                                                    (1000, 700, 0, 1), (352800, 264600, 1, 50),
                                                    (352800, 264600, 0, 50), (352800, 264600, 49, 50)])
def test_chunk_weights_closed_form(chunk, step, index, count):
    w = O.chunk_weights(chunk, step, index, count)
    ref = fade64(chunk, step, index, count)
    assert np.allclose(w, ref, rtol=0, atol=1e-7)
    ov = chunk - step
    # explicit positions: a rising edge starts at 1/(2O), a falling one ends there
    assert w[0] == (np.float32(0.5) / np.float32(ov) if index > 0 else 1.0)
    assert w[-1] == (np.float32(0.5) / np.float32(ov) if index + 1 < count else 1.0)
    assert w[ov] == 1.0 and w[chunk - ov - 1] == 1.0
    if index > 0:
        assert w[ov - 1] == np.float32(ov - 0.5) / np.float32(ov)


def test_chunked_separation_matches_numpy_composition():
    """or_separate_chunked on 4 windows with a zero-padded tail against the
    float64 statement sum_k w_k * forward(window_k) / sum_k w_k, each window
    cut by numpy at k*step (zero-padded past the end), w_k the closed-form
    fades of helpers.fade64.  Swapped fade branches or a window one step off move the
    output far outside the tolerance (checked below on the statement)."""
    d = CONFIG_DIMS.with_depth(1)
    blob = pack.synthetic_pack(d, 41)
    m = O.Model(d, blob)
    chunk, step = 4410, 3087
    length = chunk + 2 * step + 1000
    x = audio.sine_mix(length / 44100.0, 15)
    assert x.shape[1] == length
    count = O.chunk_count(length, chunk, step)
    assert count == 4 and (count - 1) * step + chunk > length

    outs = []
    for k in range(count):
        win = np.zeros((2, chunk), np.float32)
        seg = x[:, k * step:min(length, k * step + chunk)]
        win[:, :seg.shape[1]] = seg
        outs.append(m.forward(win).astype(np.float64))

    def compose(weights, starts):
        return compose_windows(outs, length, chunk, step, weights, starts)

    def sum_overlapped(weights, starts):
        den = np.zeros(length)
        for k in range(count):
            n = min(length, starts[k] + chunk) - starts[k]
            den[starts[k]:starts[k] + n] += weights[k][:n]
        return den

    starts = [k * step for k in range(count)]
    fades = [fade64(chunk, step, k, count) for k in range(count)]
    ref = compose(fades, starts)
    got = m.separate_chunked(x, chunk, step)
    scale = float(np.max(np.abs(ref)))
    tol = 1e-6 * scale
    assert np.max(np.abs(got - ref)) <= tol

    # the statement's power: planted mistakes land far outside the tolerance
    swapped = [_fade64_swapped(chunk, step, k, count) for k in range(count)]
    assert np.allclose(sum_overlapped(swapped, starts), 1.0)  # still a partition of unity
    err_swapped = np.max(np.abs(compose(swapped, starts) - ref))
    assert err_swapped > 100 * tol, err_swapped
    # window 2's output composed one sample off where it was cut
    shifted = list(starts)
    shifted[2] += 1
    err_shifted = np.max(np.abs(compose(fades, shifted) - ref))
    assert err_shifted > 100 * tol, err_shifted


def test_chunked_separation_of_one_window_is_forward():
    d = CONFIG_DIMS.with_depth(1)
    blob = pack.synthetic_pack(d, 6)
    m = O.Model(d, blob)
    x = audio.sine_mix(0.1, 1)
    assert np.array_equal(m.separate_chunked(x, x.shape[1], x.shape[1] // 2), m.forward(x))
