"""fp32 linears on bf16 matrix cores by exact operand splitting.

Every fp32 x is the exact sum of three bf16 pieces h = bf16(x),
m = bf16(x - h), l = x - h - m.  The split GEMM accumulates the six piece
products that can reach 2^-24 of |a||w| in fp32.  Pinned here:
  * the pieces: bit-identical to torch's nearest-even bf16 rounding applied
    in that chain, summing back to W exactly, at the documented tile-major
    positions (every position written once, rows past N zero);
  * the GEMM: its error against a float64 product of the fp32 operands is no
    larger than the fp32 MFMA GEMM's (max and rms), and below a hard bound of
    2^-18 * sum_k |a_k w_k| that a dropped or misplaced piece product (>= 2^-8
    relative for hm/mh, a wrong slot: O(1)) would break;
  * the model: the fp32 parity bar (max |d| <= 1e-4, SNR >= 80 dB against the
    oracle) with the split linears and with the fp32 MFMA ones.
"""

import numpy as np
import pytest

from helpers import empty_dev, from_dev, gpu_available, snr_db, to_dev

pytestmark = pytest.mark.gpu

if gpu_available():
    import torch
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


def _slot(k: np.ndarray) -> np.ndarray:
    """Position of k in its group of 16: k 0-3, 8-11 (slot 0), 4-7, 12-15 (slot 1)."""
    r = k & 15
    return (k & ~15) + 8 * ((r >> 2) & 1) + (r & 3) + 4 * (r >> 3)


def _piece_index(n: np.ndarray, k: np.ndarray, p: int, K: int) -> np.ndarray:
    """bf16 index of piece p of W[n][k] in the tile-major layout of vh_split_weights."""
    pos = _slot(k) & 15
    s, e = pos >> 3, pos & 7
    return (((n // 128) * (K // 16) + k // 16) * 3 + p) * 2048 + (n % 128) * 16 + 8 * (s ^ ((n // 8) & 1)) + e


def _bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).to(torch.float32).numpy()


def _split(ctx, w: np.ndarray):
    n, k = w.shape
    pieces = torch.zeros(ctx.split_bytes(n, k) // 2, dtype=torch.bfloat16, device="cuda:0")
    ctx.split_weights(to_dev(w), pieces, n, k)
    return pieces


def test_slot_permutation_is_a_bijection():
    k = np.arange(64)
    s = _slot(k)
    assert sorted(s.tolist()) == k.tolist()
    assert s[:16].tolist() == [0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15]


def test_split_weights_exact(ctx, rng):
    n, k = 137, 48  # two row tiles, the second ragged
    assert ctx.split_bytes(n, k) == 256 * k * 6
    w = rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.05)
    # full 24-bit significands, powers of two, signs, zeros, tiny and large values
    w[0, :8] = [1.0, -0.5, 0.0, -0.0, 3.0e38, -1.0e-30, 1.0 + 2.0 ** -23, -(1.0 - 2.0 ** -24)]
    w[1, :] = (np.arange(k, dtype=np.uint32) * 0x1F3 | 0x3F800000).view(np.float32)
    pieces = torch.full((ctx.split_bytes(n, k) // 2,), 7.0, dtype=torch.bfloat16, device="cuda:0")
    ctx.split_weights(to_dev(w), pieces, n, k)
    torch.cuda.synchronize()
    flat = pieces.float().cpu().numpy()
    nn, kk = np.meshgrid(np.arange(256), np.arange(k), indexing="ij")
    idx = [_piece_index(nn, kk, p, k) for p in range(3)]
    # every element written exactly once, rows past N zero
    assert sorted(np.concatenate([i.ravel() for i in idx]).tolist()) == list(range(flat.size))
    for p in range(3):
        assert np.all(flat[idx[p][n:]] == 0.0)
    h, m, l = (flat[idx[p][:n]] for p in range(3))
    # the rounding chain, bit for bit
    h_ref = _bf16(w)
    m_ref = _bf16(w - h_ref)
    l_ref = _bf16((w - h_ref) - m_ref)
    assert np.array_equal(h.view(np.uint32), h_ref.view(np.uint32))
    assert np.array_equal(m.view(np.uint32), m_ref.view(np.uint32))
    assert np.array_equal(l.view(np.uint32), l_ref.view(np.uint32))
    # exact reconstruction (float64 sums of the pieces are exact)
    assert np.array_equal(h.astype(np.float64) + m + l, w.astype(np.float64))


SPLIT_CASES = [
    # M, N, K, epilogue, bias
    (300, 200, 96, 0, True),
    (1000, 1568, 384, 0, True),   # ragged last column tile (1568 = 12.25 x 128)
    (4097, 768, 512, 0, False),
    (77, 384, 1536, 3, True),
    (257, 1024, 256, 1, True),
    (130, 1536, 384, 2, True),
    (1, 8, 16, 0, True),          # one K chunk, one row
    (513, 129, 32, 3, False),
]


def _ref64(x, w, b):
    y = x.astype(np.float64) @ w.astype(np.float64).T
    if b is not None:
        y += b.astype(np.float64)
    return y


@pytest.mark.parametrize("M,N,K,epi,has_bias", SPLIT_CASES)
def test_gemm_split_accuracy(ctx, rng, M, N, K, epi, has_bias):
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) * np.float32(0.1) if has_bias else None
    c0 = rng.standard_normal((M, N)).astype(np.float32)
    planes = _split(ctx, w)
    db = to_dev(b) if b is not None else None
    outs = {}
    for kind in ("split", "fp32"):
        dc = to_dev(c0)
        if kind == "split":
            ctx.gemm_split(to_dev(x), planes, dc, M, N, K, bias=db, epilogue=epi)
        else:
            ctx.gemm(to_dev(x), to_dev(w), dc, M, N, K, bias=db, epilogue=epi)
        outs[kind] = from_dev(dc).astype(np.float64)
    pre = _ref64(x, w, b)
    if epi == native.EPI_STORE or epi == native.EPI_RESIDUAL:
        ref = pre + (c0 if epi == native.EPI_RESIDUAL else 0.0)
        err = {kind: np.abs(o - ref) for kind, o in outs.items()}
        scale = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T
        bound = 2.0 ** -18 * scale + 2.0 ** -22 * np.abs(ref)
        worst = float(np.max(err["split"] - bound))
        print(f"split {M}x{N}x{K} epi{epi}: max|d| {err['split'].max():.3e} rms {np.sqrt(np.mean(err['split'] ** 2)):.3e}"
              f" | fp32 MFMA max|d| {err['fp32'].max():.3e} rms {np.sqrt(np.mean(err['fp32'] ** 2)):.3e}")
        assert worst <= 0, f"error above 2^-18 sum|a||w| by {worst:.3e}"
        assert err["split"].max() <= 1.5 * err["fp32"].max() + 1e-7
        assert np.sqrt(np.mean(err["split"] ** 2)) <= 1.25 * np.sqrt(np.mean(err["fp32"] ** 2)) + 1e-8
    else:
        # GELU / tanh epilogues: the same pre-activation, the same fp32 epilogue code
        f = (lambda v: O.gelu(v.astype(np.float32)).astype(np.float64)) if epi == native.EPI_GELU else np.tanh
        ref = f(pre)
        e_split = np.abs(outs["split"] - ref).max()
        e_fp32 = np.abs(outs["fp32"] - ref).max()
        print(f"split {M}x{N}x{K} epi{epi}: max|d| {e_split:.3e} | fp32 MFMA {e_fp32:.3e}")
        assert e_split <= 1.5 * e_fp32 + 1e-6


def test_gemm_split_geglu(ctx, rng):
    M, F, K = 333, 192, 384
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (0.05 * rng.standard_normal((2 * F, K))).astype(np.float32)
    b = (0.1 * rng.standard_normal(2 * F)).astype(np.float32)
    ref = O.geglu(_ref64(x, w, b).astype(np.float32)).astype(np.float64)
    perm = np.empty(2 * F, dtype=np.int64)  # the library's 32-row value/gate interleave
    for c in range(F):
        perm[(c // 32) * 64 + (c % 32)] = c
        perm[(c // 32) * 64 + 32 + (c % 32)] = F + c
    planes = _split(ctx, np.ascontiguousarray(w[perm]))
    dc = empty_dev((M, F))
    ctx.gemm_split(to_dev(x), planes, dc, M, 2 * F, K, bias=to_dev(np.ascontiguousarray(b[perm])),
                   epilogue=native.EPI_GEGLU)
    err = np.abs(from_dev(dc) - ref)
    assert err.max() <= 2e-5, err.max()


def test_gemm_split_rejects_bad_shapes(ctx):
    x = torch.zeros(8, 24, device="cuda:0")
    pieces = torch.zeros(ctx.split_bytes(8, 32) // 2, dtype=torch.bfloat16, device="cuda:0")
    c = torch.zeros(8, 8, device="cuda:0")
    with pytest.raises(native.NativeError, match="unsupported shape"):
        ctx.gemm_split(x, pieces, c, 8, 8, 24)  # K must be a multiple of 16
    with pytest.raises(native.NativeError, match="unsupported shape"):
        ctx.gemm_split(x, pieces, c, 8, 8, 16, lda=14)  # lda must be a multiple of 4 and >= K
    with pytest.raises(native.NativeError, match="unsupported shape"):
        ctx.gemm_split(x, pieces, c, 8, 8, 16, ldc=(1 << 21) + 8)  # ldc <= 2^21 (32-bit row offsets)
    with pytest.raises(native.NativeError, match="bad shape"):
        ctx.split_weights(torch.zeros(8, 24, device="cuda:0"), pieces, 8, 24)  # K % 16


@pytest.mark.parametrize("dims_name", ["config", "reference"])
def test_forward_split_and_fp32_mfma(ctx, ref_pack, dims_name):
    """The parity bar with the split linears (default) and with every product
    on the fp32 MFMA instruction; the two agree far inside it."""
    if dims_name == "config":
        d, blob, secs = CONFIG_DIMS.with_depth(4), None, 0.5
        blob = pack.synthetic_pack(d, 9)
    else:
        d, blob, secs = REFERENCE_DIMS, ref_pack, 0.2
    om, dm = O.Model(d, blob), native.Model(ctx, d, blob)
    x = audio.sine_mix(secs, 31)
    ref = om.forward(x)
    outs = {}
    for prec in (native.PRECISION_FP32, native.PRECISION_FP32_MFMA):
        dm.set_precision(prec)
        dv = empty_dev(x.shape)
        dm.forward(to_dev(x), x.shape[1], dv)
        outs[prec] = from_dev(dv).astype(np.float64)
        err = float(np.max(np.abs(outs[prec] - ref)))
        print(f"forward {dims_name} precision {prec}: max|d| {err:.3e}, SNR {snr_db(ref, outs[prec]):.1f} dB")
        assert err <= 1e-4
        assert snr_db(ref, outs[prec]) >= 80
    assert snr_db(outs[native.PRECISION_FP32_MFMA], outs[native.PRECISION_FP32]) >= 90
    dm.close()
