"""fp32 linears on fp16 matrix cores by two-piece operand splitting.

Each operand is scaled by a power of two 2^e that puts its bound below 2^14,
and every scaled value y is split into h = fp16(y), m = fp16(y - h) (nearest
even); the GEMM accumulates hh + hm + mh in fp32 and scales back.  Pinned here:
  * the exponent and the pieces: max|W| in the header, h and m bit-identical
    to numpy's nearest-even float16 rounding applied in that chain, at the
    documented tile-major positions (every position written once, rows past
    N zero), h + m within 2^-22 |y| (or 2^-25 absolute) of y;
  * the GEMM: its error against a float64 product of the fp32 operands is no
    larger than the fp32 MFMA GEMM's (max and rms) and below 2^-18 sum|a w|,
    which a dropped hm/mh product (2^-11 relative) or a misplaced piece would
    break; an explicit bound equal to max|A| gives the same bits as the
    computed one; a bound 2^16 times too loose still meets the error bound;
  * the operand bounds: equal to their closed forms (sqrt(D) max|gamma|,
    sqrt(D) max|gamma| max||W_n|| + max|b|, squared for GELU-GLU) and never
    exceeded by an RMSNorm output, its linear or its GELU-GLU;
  * the model: the fp32 parity bar with these linears (test_gpu_split's
    forward test runs the default path, which uses them).
"""

import numpy as np
import pytest

from helpers import empty_dev, from_dev, gpu_available, to_dev

pytestmark = pytest.mark.gpu

if gpu_available():
    import torch
    import oracle as O
    from vocalarc_hip import native


@pytest.fixture(scope="module")
def ctx():
    if not gpu_available():
        pytest.skip("no GPU")
    c = native.Context()
    yield c
    c.close()


def _slot(k: np.ndarray) -> np.ndarray:
    r = k & 15
    return (k & ~15) + 8 * ((r >> 2) & 1) + (r & 3) + 4 * (r >> 3)


def _piece_index(n: np.ndarray, k: np.ndarray, p: int, K: int) -> np.ndarray:
    """fp16 index of piece p of W[n][k] in the layout of vh_split_weights_h2 (after the 128-half header)."""
    pos = _slot(k) & 15
    s, e = pos >> 3, pos & 7
    return 128 + (((n // 128) * (K // 16) + k // 16) * 2 + p) * 2048 + (n % 128) * 16 + 8 * (s ^ ((n // 8) & 1)) + e


def _exponent(bound: float) -> int:
    """The e with bound * 2^e < 2^14, largest such (frexp: bound = f 2^E, f in [0.5, 1))."""
    if not bound > 0 or not np.isfinite(bound):
        return 0
    return int(np.clip(14 - np.frexp(np.float32(bound))[1], -100, 100))


def _pieces(ctx, w: np.ndarray):
    n, k = w.shape
    p = torch.zeros(ctx.h2_bytes(n, k) // 2, dtype=torch.float16, device="cuda:0")
    ctx.split_weights_h2(to_dev(w), p, n, k)
    return p


def test_exponent_closed_form():
    assert _exponent(1.0) == 13            # 1 * 2^13 < 2^14, 2^14 is not
    assert _exponent(0.999) == 14
    assert _exponent(16383.0) == 0
    assert _exponent(16384.0) == -1
    assert _exponent(0.0) == 0 and _exponent(float("nan")) == 0


def test_split_weights_h2_exact(ctx, rng):
    n, k = 137, 48  # two row tiles, the second ragged
    assert ctx.h2_bytes(n, k) == 256 + 256 * k * 4
    w = rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.05)
    # signs, zeros, powers of two, full significands, values far below the maximum
    w[0, :8] = [0.25, -0.125, 0.0, -0.0, 1.0e-30, -3.0e-9, 0.2 * (1 + 2.0 ** -23), -(0.1 - 2.0 ** -30)]
    w[1, :] = (np.arange(k, dtype=np.uint32) * 0x1F3 | 0x3E000000).view(np.float32)
    pieces = torch.full((ctx.h2_bytes(n, k) // 2,), 7.0, dtype=torch.float16, device="cuda:0")
    ctx.split_weights_h2(to_dev(w), pieces, n, k)
    torch.cuda.synchronize()
    raw = pieces.cpu().numpy()
    wmax = float(np.abs(w).max())
    assert raw[:2].view(np.float32)[0] == np.float32(wmax)
    flat = raw[128:].astype(np.float32)
    nn, kk = np.meshgrid(np.arange(256), np.arange(k), indexing="ij")
    idx = [_piece_index(nn, kk, p, k) - 128 for p in range(2)]
    assert sorted(np.concatenate([i.ravel() for i in idx]).tolist()) == list(range(flat.size))
    for p in range(2):
        assert np.all(flat[idx[p][n:]] == 0.0)
    h, m = (flat[idx[p][:n]] for p in range(2))
    y = w * np.float32(2.0 ** _exponent(wmax))
    assert np.abs(y).max() < 2 ** 14
    h_ref = y.astype(np.float16).astype(np.float32)
    m_ref = (y - h_ref).astype(np.float16).astype(np.float32)
    # bit for bit, except that the device may give a zero either sign
    for got, want in ((h, h_ref), (m, m_ref)):
        nz = want != 0
        assert np.array_equal(got[nz].view(np.uint32), want[nz].view(np.uint32))
        assert np.all(got[~nz] == 0.0)
    err = np.abs(h.astype(np.float64) + m - y)
    assert np.all(err <= 2.0 ** -22 * np.abs(y) + 2.0 ** -25)


CASES = [
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


@pytest.mark.parametrize("M,N,K,epi,has_bias", CASES)
def test_gemm_h2_accuracy(ctx, rng, M, N, K, epi, has_bias):
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) * np.float32(0.1) if has_bias else None
    c0 = rng.standard_normal((M, N)).astype(np.float32)
    planes = _pieces(ctx, w)
    db = to_dev(b) if b is not None else None
    dx = to_dev(x)
    amax = float(np.abs(x).max())
    outs = {}
    for kind in ("h2", "h2_bound", "h2_loose", "fp32"):
        dc = to_dev(c0)
        if kind == "fp32":
            ctx.gemm(dx, to_dev(w), dc, M, N, K, bias=db, epilogue=epi)
        else:
            bound = {"h2": 0.0, "h2_bound": amax, "h2_loose": amax * 2.0 ** 16}[kind]
            ctx.gemm_h2(dx, planes, dc, M, N, K, bias=db, epilogue=epi, a_bound=bound)
        outs[kind] = from_dev(dc).astype(np.float64)
    # the device maximum gives the same exponent as the explicit bound
    assert np.array_equal(outs["h2"], outs["h2_bound"])
    pre = _ref64(x, w, b)
    if epi == native.EPI_STORE or epi == native.EPI_RESIDUAL:
        ref = pre + (c0 if epi == native.EPI_RESIDUAL else 0.0)
        err = {kind: np.abs(o - ref) for kind, o in outs.items()}
        scale = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T
        bound = 2.0 ** -18 * scale + 2.0 ** -22 * np.abs(ref)
        for kind in ("h2", "h2_loose"):
            worst = float(np.max(err[kind] - bound))
            assert worst <= 0, f"{kind}: error above 2^-18 sum|a||w| by {worst:.3e}"
        print(f"h2 {M}x{N}x{K} epi{epi}: max|d| {err['h2'].max():.3e} rms {np.sqrt(np.mean(err['h2'] ** 2)):.3e}"
              f" | loose bound max|d| {err['h2_loose'].max():.3e}"
              f" | fp32 MFMA max|d| {err['fp32'].max():.3e} rms {np.sqrt(np.mean(err['fp32'] ** 2)):.3e}")
        if K >= 64:
            # where the fp32 accumulation over K dominates (every model shape),
            # no worse than the fp32 MFMA GEMM; for a handful of terms the
            # pieces' 2^-22 representation error shows, held by the bound above
            assert err["h2"].max() <= 1.5 * err["fp32"].max() + 1e-7
            assert np.sqrt(np.mean(err["h2"] ** 2)) <= 1.25 * np.sqrt(np.mean(err["fp32"] ** 2)) + 1e-8
        else:
            assert np.all(err["h2"] <= 2.0 ** -20 * scale + 2.0 ** -22 * np.abs(ref))
    else:
        f = (lambda v: O.gelu(v.astype(np.float32)).astype(np.float64)) if epi == native.EPI_GELU else np.tanh
        ref = f(pre)
        e_h2 = np.abs(outs["h2"] - ref).max()
        e_fp32 = np.abs(outs["fp32"] - ref).max()
        print(f"h2 {M}x{N}x{K} epi{epi}: max|d| {e_h2:.3e} | fp32 MFMA {e_fp32:.3e}")
        assert e_h2 <= 1.5 * e_fp32 + 1e-6


def test_gemm_h2_geglu(ctx, rng):
    M, F, K = 333, 192, 384
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (0.05 * rng.standard_normal((2 * F, K))).astype(np.float32)
    b = (0.1 * rng.standard_normal(2 * F)).astype(np.float32)
    ref = O.geglu(_ref64(x, w, b).astype(np.float32)).astype(np.float64)
    perm = np.empty(2 * F, dtype=np.int64)  # the library's 32-row value/gate interleave
    for c in range(F):
        perm[(c // 32) * 64 + (c % 32)] = c
        perm[(c // 32) * 64 + 32 + (c % 32)] = F + c
    planes = _pieces(ctx, np.ascontiguousarray(w[perm]))
    dc = empty_dev((M, F))
    ctx.gemm_h2(to_dev(x), planes, dc, M, 2 * F, K, bias=to_dev(np.ascontiguousarray(b[perm])),
                epilogue=native.EPI_GEGLU)
    err = np.abs(from_dev(dc) - ref)
    assert err.max() <= 2e-5, err.max()


@pytest.mark.parametrize("S,L", [(3, 801), (2, 97), (40, 62), (30, 17)])
def test_attention_h2_rows_out(ctx, rng, S, L):
    """VH_ATT_OUT_H2: the two-piece attention (time-axis kernel for L > 64,
    band-axis kernel otherwise) writes its output as h2 rows scaled from
    max|qkv|: the pieces are those of its fp32 output times 2^e, bit for bit,
    at the documented positions, and the out projection fed them gives the
    same bits as the GEMM splitting that fp32 output itself with the same
    bound.  Ragged lengths leave rows of the last query wave partly empty."""
    H, N = 8, 384
    K = H * 64
    qkv = rng.standard_normal((S * L, 3 * K)).astype(np.float32)
    dq = to_dev(qkv)
    bound = float(np.abs(qkv).max())
    out32 = empty_dev((S * L, K))
    outh = torch.full((S * L, K), 7.0, device="cuda:0")
    ctx.attention(dq, out32, S, L, H, rotary=True, h2=True)
    ctx.attention(dq, outh, S, L, H, rotary=True, h2=True, out_h2=True)
    torch.cuda.synchronize()
    y = from_dev(out32)
    e = _exponent(bound)
    h, m = _decode_h2_rows(outh.cpu().numpy().view(np.float16).ravel(), S * L, K)
    ys = y * np.float32(2.0 ** e)
    h_ref = ys.astype(np.float16).astype(np.float32)
    m_ref = (ys - h_ref).astype(np.float16).astype(np.float32)
    for got, want in ((h, h_ref), (m, m_ref)):
        nz = want != 0
        assert np.array_equal(got[nz].view(np.uint32), want[nz].view(np.uint32))
        assert np.all(got[~nz] == 0.0)
    w = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    planes = _pieces(ctx, w)
    c_rows, c_fp32 = to_dev(np.ones((S * L, N), np.float32)), to_dev(np.ones((S * L, N), np.float32))
    ctx.gemm_h2(outh, planes, c_rows, S * L, N, K, epilogue=native.EPI_RESIDUAL, a_bound=bound, a_rows=True)
    ctx.gemm_h2(out32, planes, c_fp32, S * L, N, K, epilogue=native.EPI_RESIDUAL, a_bound=bound)
    torch.cuda.synchronize()
    assert torch.equal(c_rows, c_fp32)
    with pytest.raises(native.NativeError):
        ctx.attention(dq, outh, S, L, H, rotary=True, out_h2=True)  # h2 rows need the two-piece kernel


def _geglu_perm(F: int) -> np.ndarray:
    """Row order of a GELU-GLU weight in the library: 32 value rows, then their 32 gate rows."""
    perm = np.empty(2 * F, dtype=np.int64)
    for c in range(F):
        perm[(c // 32) * 64 + (c % 32)] = c
        perm[(c // 32) * 64 + 32 + (c % 32)] = F + c
    return perm


@pytest.mark.parametrize("epi", ["store", "geglu", "gelu"])
def test_gemm_h2_row_norm(ctx, rng, epi):
    """The GEMM of an RMSNorm of x's rows (VH_H2_ROW_NORM): x raw, the gain
    folded into the weight's pieces, each output row scaled by
    sqrt(D) / sqrt(sum x^2 + 1e-12) inside the GEMM.  Against a float64
    RMSNorm and linear of the same fp32 inputs, with the bound max|x| (what
    the model passes), its error is as small as that of the unfused pair
    (fp32 RMSNorm kernel, then the two-piece GEMM) and within 2^-18
    sum|y||w|; a dropped or misplaced row scale would be off by the rows'
    norms (the rows' scales span e^+-3).  With a bound 2^10 times looser the
    pieces of x are exact only to 2^-25 / 2^e absolute (e from the bound), so
    a row's error grows with its scale factor: held to that analytic bound.
    Rows are ragged against the 256-row tile."""
    rows, D = 1000, 384
    N = {"store": 1568, "geglu": 2 * 192, "gelu": 256}[epi]
    code = {"store": native.EPI_STORE, "geglu": native.EPI_GEGLU, "gelu": native.EPI_GELU}[epi]
    x = (rng.standard_normal((rows, D)) * np.exp(rng.standard_normal((rows, 1)))).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    w = (0.05 * rng.standard_normal((N, D))).astype(np.float32)
    b = (0.1 * rng.standard_normal(N)).astype(np.float32)
    if epi == "geglu":
        perm = _geglu_perm(N // 2)
        w, b = np.ascontiguousarray(w[perm]), np.ascontiguousarray(b[perm])
    x64 = x.astype(np.float64)
    y64 = x64 * (np.sqrt(D) / np.sqrt(np.sum(x64 * x64, axis=1, keepdims=True) + 1e-12)) * gamma
    pre = y64 @ w.astype(np.float64).T + b
    if epi == "store":
        ref = pre
    elif epi == "gelu":
        ref = O.gelu(pre.astype(np.float32)).astype(np.float64)
    else:
        inv = np.argsort(perm)
        ref = O.geglu(pre[:, inv].astype(np.float32)).astype(np.float64)
    folded = _pieces(ctx, (w * gamma[None, :]).astype(np.float32))
    dx, db = to_dev(x), to_dev(b)
    cols = N // 2 if epi == "geglu" else N
    amax = float(np.abs(x).max())
    outs = {}
    loose = amax * 2.0 ** 10
    for kind, bound in (("fused", amax), ("fused_loose", loose)):
        dbound = torch.tensor([bound], dtype=torch.float32, device="cuda:0")
        zero = torch.tensor([5.0], device="cuda:0")
        dc = empty_dev((rows, cols))
        ctx.gemm_h2_ex(dx, folded, dc, rows, N, D, dbound, bias=db, epilogue=code, row_norm=True, zero_slot=zero)
        torch.cuda.synchronize()
        assert float(zero.cpu()[0]) == 0.0
        outs[kind] = from_dev(dc).astype(np.float64)
    # the unfused pair on the same inputs
    dy = empty_dev((rows, D))
    ctx.rmsnorm(dx, to_dev(gamma), dy, rows, D)
    dc = empty_dev((rows, cols))
    ctx.gemm_h2(dy, _pieces(ctx, w), dc, rows, N, D, bias=db, epilogue=code)
    outs["unfused"] = from_dev(dc).astype(np.float64)
    err = {k: np.abs(o - ref) for k, o in outs.items()}
    print(f"row norm {epi}: fused max|d| {err['fused'].max():.3e} rms {np.sqrt(np.mean(err['fused'] ** 2)):.3e}"
          f" | loose {err['fused_loose'].max():.3e} | unfused max|d| {err['unfused'].max():.3e}"
          f" rms {np.sqrt(np.mean(err['unfused'] ** 2)):.3e}")
    assert err["fused"].max() <= 1.5 * err["unfused"].max() + 1e-7
    assert np.sqrt(np.mean(err["fused"] ** 2)) <= 1.25 * np.sqrt(np.mean(err["unfused"] ** 2)) + 1e-8
    if epi == "store":
        aw = np.abs(w.astype(np.float64))
        scale = np.abs(y64) @ aw.T
        assert np.all(err["fused"] <= 2.0 ** -18 * scale + 2.0 ** -22 * np.abs(ref))
        # loose bound: each x element carries up to 2^-24 / 2^e absolute more,
        # times the row's scale factor and |gamma_k w_nk| summed over k
        r = np.sqrt(D) / np.sqrt(np.sum(x64 * x64, axis=1, keepdims=True) + 1e-12)
        extra = r * 2.0 ** (-24 - _exponent(loose)) * (np.abs(gamma.astype(np.float64)) @ aw.T)[None, :]
        assert np.all(err["fused_loose"] <= 2.0 ** -18 * scale + 2.0 ** -22 * np.abs(ref) + extra)
    # the fp32 bar against the oracle's RMSNorm and linear
    assert err["fused"].max() <= 2e-5 * max(1.0, float(np.abs(ref).max()))


def test_gemm_h2_residual_amax(ctx, rng):
    """The residual epilogue's amax: raised to exactly max |C| over the
    elements written (the fp32 values stored), from below and not lowered
    from above; the bound the next row-norm GEMM splits the residual stream
    with.  Rows ragged against the tile, N = 384 (three column tiles)."""
    M, N, K = 1000, 384, 512
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    c0 = (3.0 * rng.standard_normal((M, N))).astype(np.float32)
    planes = _pieces(ctx, w)
    dbound = torch.tensor([float(np.abs(x).max())], device="cuda:0")
    for start in (0.0, 1.0e6):
        amax = torch.tensor([start], device="cuda:0")
        dc = to_dev(c0)
        ctx.gemm_h2_ex(to_dev(x), planes, dc, M, N, K, dbound, epilogue=native.EPI_RESIDUAL, amax=amax)
        torch.cuda.synchronize()
        want = max(start, float(dc.abs().max().cpu()))
        assert float(amax.cpu()[0]) == want, (start, float(amax.cpu()[0]), want)
    with pytest.raises(native.NativeError):
        ctx.gemm_h2_ex(to_dev(x), planes, empty_dev((M, N)), M, N, K, dbound, epilogue=native.EPI_STORE, amax=amax)
    with pytest.raises(native.NativeError):
        ctx.gemm_h2_ex(to_dev(x), planes, empty_dev((M, N)), M, N, K, dbound, epilogue=native.EPI_RESIDUAL,
                       row_norm=True)
    # every workgroup reads the bound while tile 0 zeroes zero_slot and the
    # epilogues raise amax: neither may be the bound itself (host-side check,
    # nothing launched)
    with pytest.raises(native.NativeError, match="alias"):
        ctx.gemm_h2_ex(to_dev(x), planes, to_dev(c0), M, N, K, dbound, epilogue=native.EPI_RESIDUAL, amax=dbound)
    with pytest.raises(native.NativeError, match="alias"):
        ctx.gemm_h2_ex(to_dev(x), planes, empty_dev((M, N)), M, N, K, dbound, epilogue=native.EPI_STORE,
                       zero_slot=dbound)


@pytest.mark.parametrize("epi_name", ["store", "residual", "geglu"])
def test_gemm_h2_padded_c(ctx, rng, epi_name):
    """C with a row pitch wider than its columns (ldc = out + 24): full row
    tiles store through a wave-uniform row pointer plus a lane offset, the
    last (ragged) row tile per element; both must give the compact result's
    bits in the first columns and leave the padding as it was."""
    epi = {"store": native.EPI_STORE, "residual": native.EPI_RESIDUAL, "geglu": native.EPI_GEGLU}[epi_name]
    M, N, K = 700, 384, 128
    out = N // 2 if epi == native.EPI_GEGLU else N
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    b = to_dev((0.1 * rng.standard_normal(N)).astype(np.float32))
    planes = _pieces(ctx, w)
    c0 = rng.standard_normal((M, out + 24)).astype(np.float32)
    compact = to_dev(np.ascontiguousarray(c0[:, :out]))
    padded = to_dev(c0)
    dx = to_dev(x)
    ctx.gemm_h2(dx, planes, compact, M, N, K, bias=b, epilogue=epi, a_bound=float(np.abs(x).max()))
    ctx.gemm_h2(dx, planes, padded, M, N, K, bias=b, epilogue=epi, ldc=out + 24, a_bound=float(np.abs(x).max()))
    got = from_dev(padded)
    assert np.array_equal(got[:, :out].view(np.uint32), from_dev(compact).view(np.uint32))
    assert np.array_equal(got[:, out:].view(np.uint32), c0[:, out:].view(np.uint32)), "padding columns were written"


def test_gemm_h2_rejects_bad_shapes(ctx):
    x = torch.zeros(8, 24, device="cuda:0")
    pieces = torch.zeros(ctx.h2_bytes(8, 32) // 2, dtype=torch.float16, device="cuda:0")
    c = torch.zeros(8, 8, device="cuda:0")
    with pytest.raises(native.NativeError, match="unsupported shape"):
        ctx.gemm_h2(x, pieces, c, 8, 8, 24, a_bound=1.0)  # K must be a multiple of 16
    with pytest.raises(native.NativeError, match="unsupported shape"):
        ctx.gemm_h2(x, pieces, c, 8, 8, 16, lda=14, a_bound=1.0)  # lda must be a multiple of 4 and >= K
    with pytest.raises(native.NativeError, match="unsupported shape"):
        ctx.gemm_h2(x, pieces, c, 8, 8, 16, ldc=(1 << 21) + 8, a_bound=1.0)  # ldc <= 2^21 (32-bit row offsets)
    with pytest.raises(native.NativeError, match="bad shape"):
        ctx.split_weights_h2(torch.zeros(8, 24, device="cuda:0"), pieces, 8, 24)  # K % 16


@pytest.mark.parametrize("square", [False, True])
def test_operand_bounds(ctx, rng, square):
    D, N, T = 384, 520, 2000
    gamma = (1.0 + 0.3 * rng.standard_normal(D)).astype(np.float32)
    w = (0.05 * rng.standard_normal((N, D))).astype(np.float32)
    b = (0.2 * rng.standard_normal(N)).astype(np.float32)
    out = torch.zeros(2, device="cuda:0")
    ctx.operand_bounds(to_dev(gamma), D, out, W=to_dev(w), N=N, bias=to_dev(b), square=square)
    got = from_dev(out).astype(np.float64)
    b0 = np.sqrt(D) * np.abs(gamma).max()
    eps = 2.0 ** -10  # the kernel's allowance for its own rounding, applied at each step
    assert abs(got[0] / (b0 * (1 + eps)) - 1) < 1e-6
    t_ref = (b0 * (1 + eps) * np.sqrt((w.astype(np.float64) ** 2).sum(1)).max() + np.abs(b).max()) * (1 + eps)
    assert abs(got[1] / (t_ref ** 2 if square else t_ref) - 1) < 1e-5
    # the bounds hold for RMSNorm outputs, their linear and its GELU-GLU --
    # including rows built to reach them (all mass on the largest gain)
    x = rng.standard_normal((T, D)).astype(np.float32) * np.exp(rng.standard_normal((T, 1))).astype(np.float32)
    x[0] = 0.0
    x[0, np.argmax(np.abs(gamma))] = 5.0
    y = O.rms_norm(x, gamma)
    assert np.abs(y).max() <= got[0]
    assert np.abs(y).max() >= 0.99 * got[0] / (1 + 2.0 ** -10)  # reached by row 0: the bound is tight
    z = y.astype(np.float64) @ w.astype(np.float64).T + b
    assert np.abs(z).max() <= (np.sqrt(got[1]) if square else got[1])
    if square:
        g = O.geglu(z.astype(np.float32))  # value = first half, gate = second half
        assert np.abs(g).max() <= got[1]
    no_w = torch.full((2,), 7.0, device="cuda:0")
    ctx.operand_bounds(to_dev(gamma), D, no_w)
    assert from_dev(no_w)[1] == 0.0


def _decode_h2_rows(raw: np.ndarray, rows: int, dim: int) -> tuple[np.ndarray, np.ndarray]:
    """h, m [rows][dim] from h2 rows (fp16 view of the buffer, 2*dim halves per row)."""
    r = raw.reshape(rows, dim // 16, 32)
    k = np.arange(16)
    pos = _slot(k)  # position of k inside its 16: slot 8*s + element e
    return r[:, :, pos].reshape(rows, dim).astype(np.float32), r[:, :, 16 + pos].reshape(rows, dim).astype(np.float32)


def test_rmsnorm_h2_rows_and_gemm(ctx, rng):
    """The RMSNorm's h2 rows are the fp16 pieces of the fp32 RMSNorm output
    times 2^e (e from the gain bound), at the documented positions; a GEMM
    fed those rows gives the same bits as the GEMM splitting the fp32 output
    itself with the same bound."""
    rows, D, N = 1000, 384, 1568
    x = (rng.standard_normal((rows, D)) * np.exp(rng.standard_normal((rows, 1)))).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    dx, dg = to_dev(x), to_dev(gamma)
    bound = torch.zeros(2, device="cuda:0")
    ctx.operand_bounds(dg, D, bound)
    y = empty_dev((rows, D))
    ctx.rmsnorm(dx, dg, y, rows, D)
    yh = torch.full((rows, D), 7.0, device="cuda:0")
    ctx.rmsnorm_h2(dx, dg, bound, yh, rows, D)
    torch.cuda.synchronize()
    b = float(from_dev(bound)[0])
    yf = from_dev(y)
    assert np.abs(yf).max() <= b
    e = _exponent(b)
    h, m = _decode_h2_rows(yh.cpu().numpy().view(np.float16).ravel(), rows, D)
    ys = yf * np.float32(2.0 ** e)
    h_ref = ys.astype(np.float16).astype(np.float32)
    m_ref = (ys - h_ref).astype(np.float16).astype(np.float32)
    for got, want in ((h, h_ref), (m, m_ref)):
        nz = want != 0
        assert np.array_equal(got[nz].view(np.uint32), want[nz].view(np.uint32))
        assert np.all(got[~nz] == 0.0)
    # the GEMM on the rows equals the GEMM splitting the fp32 values itself
    w = (0.05 * rng.standard_normal((N, D))).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    planes, db = _pieces(ctx, w), to_dev(bias)
    c_rows, c_fp32 = empty_dev((rows, N)), empty_dev((rows, N))
    ctx.gemm_h2(yh, planes, c_rows, rows, N, D, bias=db, a_bound=b, a_rows=True)
    ctx.gemm_h2(y, planes, c_fp32, rows, N, D, bias=db, a_bound=b)
    torch.cuda.synchronize()
    assert torch.equal(c_rows, c_fp32)
    with pytest.raises(native.NativeError, match="bound"):
        ctx.gemm_h2(yh, planes, c_rows, rows, N, D, a_rows=True)  # rows need the bound they were split with

