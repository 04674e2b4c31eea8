"""HIP kernels vs the oracle, through the vocalarc_hip.h C-ABI.

Tolerances (fp32 path): GEMM / norms / attention compare against the oracle's
reference-order FMA chains, so differences are summation-order rounding:
rtol 2e-5 relative to the output scale.  Elementwise kernels (rotary,
GELU-GLU, residual) are within a few ulps.
"""

import numpy as np
import pytest

from helpers import assert_close, empty_dev, from_dev, gpu_available, snr_db, to_dev

pytestmark = pytest.mark.gpu

if gpu_available():
    import torch
    import oracle as O
    from vocalarc_hip import native, pack
    from vocalarc_hip.dims import CONFIG_DIMS, REFERENCE_DIMS


@pytest.fixture(scope="module")
def ctx():
    if not gpu_available():
        pytest.skip("no GPU")
    c = native.Context()
    yield c
    c.close()


def _interleave_glu_rows(w: np.ndarray) -> np.ndarray:
    """[2F][K] value|gate rows -> the library's 32-row interleave."""
    two_f = w.shape[0]
    f = two_f // 2
    out = np.empty_like(w)
    for c in range(f):
        out[(c // 32) * 64 + (c % 32)] = w[c]
        out[(c // 32) * 64 + 32 + (c % 32)] = w[f + c]
    return out


GEMM_CASES = [
    # M, N, K, epilogue, bias
    (300, 200, 96, 0, True),
    (1000, 1536, 384, 0, False),
    (257, 1024, 256, 1, True),
    (77, 384, 1536, 3, True),
    (50, 16, 1536, 0, True),
    (40, 256, 516, 0, True),
    (33, 8, 256, 0, True),
    (130, 1536, 384, 2, True),
    (1, 32, 8, 0, True),
    (4097, 768, 384, 0, True),
]


@pytest.mark.parametrize("M,N,K,epi,has_bias", GEMM_CASES)
def test_gemm_matches_oracle(ctx, rng, M, N, K, epi, has_bias):
    x = rng.standard_normal((M, K), dtype=np.float32)
    w = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) if has_bias else None
    ref = O.matmul(x, pack.pack_matrix(w), N, b)
    if epi == native.EPI_GELU:
        ref = O.gelu(ref)
    elif epi == native.EPI_TANH:
        ref = np.tanh(ref.astype(np.float64)).astype(np.float32)
    c0 = rng.standard_normal((M, N), dtype=np.float32)
    if epi == native.EPI_RESIDUAL:
        ref = c0 + ref
    dx, dw = to_dev(x), to_dev(w)
    db = to_dev(b) if b is not None else None
    dc = to_dev(c0)
    ctx.gemm(dx, dw, dc, M, N, K, bias=db, epilogue=epi)
    out = from_dev(dc)
    scale = float(np.sqrt(K)) * 0.05 * 4 + 1.0
    assert_close(ref, out, rtol=2e-5, atol=2e-5 * scale, what=f"gemm {M}x{N}x{K} epi{epi}")


def test_gemm_geglu_epilogue(ctx, rng):
    M, F, K = 190, 1536, 384
    x = rng.standard_normal((M, K), dtype=np.float32)
    w = (0.05 * rng.standard_normal((2 * F, K))).astype(np.float32)
    b = rng.standard_normal(2 * F).astype(np.float32)
    ref = O.geglu(O.matmul(x, pack.pack_matrix(w), 2 * F, b))
    wi = _interleave_glu_rows(w)
    bi = _interleave_glu_rows(b[:, None])[:, 0].copy()
    dc = empty_dev((M, F))
    ctx.gemm(to_dev(x), to_dev(wi), dc, M, 2 * F, K, bias=to_dev(bi), epilogue=native.EPI_GEGLU)
    assert_close(ref, from_dev(dc), rtol=2e-5, atol=5e-5, what="gemm geglu")


@pytest.mark.parametrize("rows,dim", [(1, 8), (333, 384), (1000, 256), (64, 516), (49662, 384)])
def test_rmsnorm(ctx, rng, rows, dim):
    x = rng.standard_normal((rows, dim), dtype=np.float32)
    g = (1.0 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
    ref = O.rms_norm(x, g)
    dy = empty_dev((rows, dim))
    ctx.rmsnorm(to_dev(x), to_dev(g), dy, rows, dim)
    assert_close(ref, from_dev(dy), rtol=4e-6, atol=1e-6, what=f"rmsnorm {rows}x{dim}")


@pytest.mark.parametrize("rows,length", [(7, 801), (100, 62), (3, 1), (5, 2048), (2000, 801), (9, 1000), (6, 4092)])
def test_softmax_rows(ctx, rng, rows, length):
    x = (3.0 * rng.standard_normal((rows, length))).astype(np.float32)
    ref = O.softmax_rows(x)
    dy = empty_dev((rows, length))
    ctx.softmax_rows(to_dev(x), dy, rows, length)
    out = from_dev(dy)
    assert_close(ref, out, rtol=1e-5, atol=1e-9, what="softmax")
    assert np.allclose(out.astype(np.float64).sum(-1), 1.0, atol=1e-5)


@pytest.mark.parametrize("b,length", [(62, 801), (801, 62), (3, 5)])
def test_rope_bhld(ctx, rng, b, length):
    x = rng.standard_normal((b, 8, length, 64), dtype=np.float32)
    ref = O.rope_bhld(x)
    dx = to_dev(x)
    ctx.rope_bhld(dx, b * 8, length)
    out = from_dev(dx)
    assert_close(ref, out, rtol=1e-6, atol=1e-6, what="rope")
    # rotation preserves the norm of each pair
    n_in = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    n_out = out[..., 0::2].astype(np.float64) ** 2 + out[..., 1::2] ** 2
    assert np.allclose(n_in, n_out, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("rows,width", [(49662, 1536), (7, 4)])
def test_geglu(ctx, rng, rows, width):
    x = rng.standard_normal((rows, 2 * width), dtype=np.float32)
    ref = O.geglu(x)
    dy = empty_dev((rows, width))
    ctx.geglu(to_dev(x), dy, rows, width)
    # 1 + erf(g/sqrt2) cancels for strongly negative gates, so the few-ulp
    # difference between the device and libm erff is bounded in absolute
    # terms (outputs are O(1) here), not relative ones.
    assert_close(ref, from_dev(dy), rtol=2e-6, atol=2e-6, what="geglu")


def test_gelu_accuracy_sweep(ctx):
    """The device GELU (polynomial-in-t erf form) against float64 over a dense
    sweep of [-10, 10]: within 1.5e-7 * max(|x|, 1), what a GELU built on a
    correctly rounded fp32 erf achieves (1.04e-7 over the same sweep)."""
    from scipy.special import erf
    g = np.linspace(-10.0, 10.0, 1 << 20).astype(np.float32)
    g[:4] = [0.0, -0.0, 1e-30, -1e-30]
    x = np.empty((1, 2 * g.size), np.float32)
    x[0, :g.size] = 1.0  # value half: GELU-GLU then returns GELU(gate)
    x[0, g.size:] = g
    dy = empty_dev((1, g.size))
    ctx.geglu(to_dev(x), dy, 1, g.size)
    out = from_dev(dy)[0].astype(np.float64)
    gd = g.astype(np.float64)
    ref = 0.5 * gd * (1.0 + erf(gd / np.sqrt(2.0)))
    err = np.abs(out - ref) / np.maximum(np.abs(gd), 1.0)
    print(f"GELU sweep: max |d| / max(|x|, 1) = {err.max():.3e}")
    assert err.max() <= 1.5e-7
    assert np.all(out[gd < -9.5] <= 0) and np.all(np.abs(out[gd > 9.5] - gd[gd > 9.5]) <= 2e-6)


def test_residual_add(ctx, rng):
    n = 49662 * 384
    x = rng.standard_normal(n, dtype=np.float32)
    r = rng.standard_normal(n, dtype=np.float32)
    dx = to_dev(x)
    ctx.residual_add(dx, to_dev(r), n)
    assert np.array_equal(from_dev(dx), x + r)


def _rotate_qk(qkv: np.ndarray, length: int, heads: int) -> np.ndarray:
    cos, sin = O.rope_table(length, 64)
    out = qkv.copy()
    tokens = qkv.shape[0]
    pos = np.arange(tokens) % length
    inner = heads * 64
    for which in range(2):
        blk = out[:, which * inner:(which + 1) * inner].reshape(tokens, heads, 32, 2)
        a, b = blk[..., 0].copy(), blk[..., 1].copy()
        c, s = cos[pos][:, None, :], sin[pos][:, None, :]
        blk[..., 0] = a * c - b * s
        blk[..., 1] = a * s + b * c
        out[:, which * inner:(which + 1) * inner] = blk.reshape(tokens, inner)
    return out


@pytest.mark.parametrize("S,L", [(5, 62), (2, 801), (3, 33), (4, 1), (1, 65), (2, 130), (7, 64), (2, 17)])
def test_attention_core(ctx, rng, S, L):
    H = 8
    qkv = rng.standard_normal((S * L, 3 * H * 64), dtype=np.float32)
    ref = O.attention(REFERENCE_DIMS, _rotate_qk(qkv, L, H), S, L)
    dout = empty_dev((S * L, H * 64))
    ctx.attention(to_dev(qkv), dout, S, L, H, rotary=True)
    out = from_dev(dout)
    assert_close(ref, out, rtol=2e-5, atol=2e-5, what=f"attention S={S} L={L}")
    assert snr_db(ref, out) > 100


@pytest.mark.parametrize("S,L", [(2, 801), (1, 65), (2, 130), (3, 97), (1, 1000)])
@pytest.mark.parametrize("mode", ["split", "h2"])
def test_attention_split(ctx, rng, S, L, mode):
    """Time-axis attention with both products in fp32 accuracy on the matrix
    cores -- exact three-piece bf16 splits (split) or two-piece fp16 splits of
    power-of-two-scaled operands (h2, the default path's kernel): the fp32 bar
    against the oracle, and an error against a float64 statement no larger
    than the fp32 MFMA kernel's on the same inputs."""
    H = 8
    qkv = rng.standard_normal((S * L, 3 * H * 64), dtype=np.float32)
    rot = _rotate_qk(qkv, L, H)
    ref = O.attention(REFERENCE_DIMS, rot, S, L)
    # float64 attention of the same rotated fp32 inputs
    q = rot[:, :H * 64].reshape(S, L, H, 64).astype(np.float64)
    k = rot[:, H * 64:2 * H * 64].reshape(S, L, H, 64).astype(np.float64)
    v = rot[:, 2 * H * 64:].reshape(S, L, H, 64).astype(np.float64)
    sc = np.einsum("slhd,smhd->shlm", q, k) * 0.125
    p = np.exp(sc - sc.max(axis=-1, keepdims=True))
    ref64 = np.einsum("shlm,smhd->slhd", p / p.sum(axis=-1, keepdims=True), v).reshape(S * L, H * 64)
    outs = {}
    for kind in (mode, "fp32"):
        dout = empty_dev((S * L, H * 64))
        ctx.attention(to_dev(qkv), dout, S, L, H, rotary=True, split=kind == "split", h2=kind == "h2")
        outs[kind] = from_dev(dout).astype(np.float64)
    assert_close(ref, outs[mode].astype(np.float32), rtol=2e-5, atol=2e-5, what=f"{mode} attention S={S} L={L}")
    e_split, e_fp32 = np.abs(outs[mode] - ref64), np.abs(outs["fp32"] - ref64)
    print(f"attention S={S} L={L}: {mode} max|d| {e_split.max():.3e} rms {np.sqrt(np.mean(e_split ** 2)):.3e} | "
          f"fp32 MFMA max|d| {e_fp32.max():.3e} rms {np.sqrt(np.mean(e_fp32 ** 2)):.3e}")
    # the rms pins the error level; the single worst element of ~10^6 is a
    # noisier statistic and gets a looser factor
    assert np.sqrt(np.mean(e_split ** 2)) <= 1.25 * np.sqrt(np.mean(e_fp32 ** 2)) + 1e-9
    assert e_split.max() <= 2.0 * e_fp32.max() + 1e-8


@pytest.mark.parametrize("S,L", [(300, 62), (200, 64), (50, 1), (90, 17), (70, 33), (40, 63)])
def test_attention_short_h2(ctx, rng, S, L):
    """Band-axis attention (L <= 64: the persistent short kernel) with both
    products as two-piece fp16 splits of power-of-two-scaled operands, the
    default path's kernel: the fp32 bar against the oracle, and an error
    against a float64 statement of the same rotated inputs no larger than the
    fp32 MFMA kernel's (ragged lengths: keys past L masked, queries past L
    not stored)."""
    H = 8
    qkv = rng.standard_normal((S * L, 3 * H * 64), dtype=np.float32)
    rot = _rotate_qk(qkv, L, H)
    ref = O.attention(REFERENCE_DIMS, rot, S, L)
    q = rot[:, :H * 64].reshape(S, L, H, 64).astype(np.float64)
    k = rot[:, H * 64:2 * H * 64].reshape(S, L, H, 64).astype(np.float64)
    v = rot[:, 2 * H * 64:].reshape(S, L, H, 64).astype(np.float64)
    sc = np.einsum("slhd,smhd->shlm", q, k) * 0.125
    p = np.exp(sc - sc.max(axis=-1, keepdims=True))
    ref64 = np.einsum("shlm,smhd->slhd", p / p.sum(axis=-1, keepdims=True), v).reshape(S * L, H * 64)
    outs = {}
    for kind in ("h2", "fp32"):
        dout = empty_dev((S * L, H * 64))
        ctx.attention(to_dev(qkv), dout, S, L, H, rotary=True, h2=kind == "h2")
        outs[kind] = from_dev(dout).astype(np.float64)
    assert_close(ref, outs["h2"].astype(np.float32), rtol=2e-5, atol=2e-5, what=f"h2 short attention S={S} L={L}")
    e_h2, e_fp32 = np.abs(outs["h2"] - ref64), np.abs(outs["fp32"] - ref64)
    print(f"short attention S={S} L={L}: h2 max|d| {e_h2.max():.3e} rms {np.sqrt(np.mean(e_h2 ** 2)):.3e} | "
          f"fp32 MFMA max|d| {e_fp32.max():.3e} rms {np.sqrt(np.mean(e_fp32 ** 2)):.3e}")
    if L == 1:
        # one key: the output is v itself, exact in fp32 and within the
        # two-piece representation's 2^-22 relative error in h2
        assert e_fp32.max() == 0.0
        assert e_h2.max() <= 2.0 ** -22 * np.abs(v).max()
        return
    assert np.sqrt(np.mean(e_h2 ** 2)) <= 1.25 * np.sqrt(np.mean(e_fp32 ** 2)) + 1e-9
    assert e_h2.max() <= 2.0 * e_fp32.max() + 1e-8


@pytest.mark.parametrize("S,L", [(2, 801), (40, 62)])
def test_attention_h2_outside_scale_range(ctx, rng, S, L):
    """VH_ATT_H2 on a qkv whose maximum (v scaled by 1e25; q, k unscaled) lies
    beyond the fp16 two-piece attention's range [2^-40, 2^60]: with one
    unscale 2^-(ek+eq) = 2^142 the scores would be inf * 0 = NaN, so the
    products run on the kernels without piece scales and the output is the
    oracle's at the fp32 bar (relative to its 1e25 scale)."""
    H = 8
    qkv = rng.standard_normal((S * L, 3 * H * 64), dtype=np.float32)
    qkv[:, 2 * H * 64:] *= np.float32(1e25)
    ref = O.attention(REFERENCE_DIMS, _rotate_qk(qkv, L, H), S, L)
    dout = empty_dev((S * L, H * 64))
    ctx.attention(to_dev(qkv), dout, S, L, H, rotary=True, h2=True)
    out = from_dev(dout)
    assert np.all(np.isfinite(out))
    assert_close(ref, out, rtol=2e-5, atol=2e-5 * 1e25, min_snr=100, what=f"h2 attention, bound 1e25, L={L}")


@pytest.mark.parametrize("mode", ["split", "h2"])
def test_attention_split_beyond_4gb(ctx, mode):
    """qkv larger than 4 GB takes the kernel's 64-bit staging addresses: its
    outputs equal, bit for bit, those of the 32-bit-offset kernel on the same
    sequences copied into a small buffer (first and last sequences).  For h2
    the scales come from each buffer's own maximum, which may differ by a
    power of two between the two buffers and with it the pieces' rounding:
    there the outputs agree to 1e-5 relative instead."""
    import torch
    S, L, H = 875, 801, 8  # 700875 rows x 6 KB = 4.31 GB > 2^32 bytes
    g = torch.Generator(device="cuda:0")
    g.manual_seed(7)
    qkv = torch.randn(S * L, 3 * H * 64, device="cuda:0", generator=g)
    assert qkv.numel() * 4 > 2 ** 32
    out = torch.empty(S * L, H * 64, device="cuda:0")
    ctx.attention(qkv, out, S, L, H, rotary=True, split=mode == "split", h2=mode == "h2")
    for first in (0, S - 2):
        small = qkv[first * L:(first + 2) * L].clone()
        ref = torch.empty(2 * L, H * 64, device="cuda:0")
        ctx.attention(small, ref, 2, L, H, rotary=True, split=mode == "split", h2=mode == "h2")
        torch.cuda.synchronize()
        if mode == "h2":
            assert torch.allclose(out[first * L:(first + 2) * L], ref, rtol=1e-5, atol=1e-6), f"sequences {first}"
            continue
        assert torch.equal(out[first * L:(first + 2) * L], ref), f"sequences {first}, {first + 1}"
    del qkv, out
    torch.cuda.empty_cache()
