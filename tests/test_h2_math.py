"""The arithmetic behind the fp16 two-piece products, checked on the CPU.

The GPU tests compare the kernels with float64; these pin the derivation the
kernels rely on, independently of any device:
  * the exponent rule and the split's error bound: for y = x 2^e with
    |x| <= B and B 2^e < 2^14, h = fp16(y), m = fp16(y - h) (nearest even)
    never overflow, y - h is exact in fp32, and |y - h - m| <= 2^-22 |y| +
    2^-25 across every binade;
  * the three-product sum: a float64 emulation of hh + hm + mh per term is
    within 2^-20 |a w| of a w, and dropping hm (a plausible slip) is not;
  * the operand bounds: an RMSNorm output never exceeds sqrt(D) max|gamma|
    and a row with all its mass on the largest gain reaches it; a linear of
    it never exceeds sqrt(D) max|gamma| max_n ||W_n|| + max|b|; a GELU-GLU of
    two such outputs never exceeds the square (|gelu(g)| <= |g|).
"""

import numpy as np

import oracle as O


def _exponent(bound: float) -> int:
    if not bound > 0 or not np.isfinite(bound):
        return 0
    return int(np.clip(14 - np.frexp(np.float32(bound))[1], -100, 100))


def _split(y: np.ndarray):
    y = y.astype(np.float32)
    h = y.astype(np.float16).astype(np.float32)
    r = (y - h).astype(np.float32)
    m = r.astype(np.float16).astype(np.float32)
    return h, m, r


def test_exponent_rule_and_split_error(rng):
    for bound in (3.0e-20, 1.0e-7, 0.37, 1.0, 19.6, 4096.0, 1.0e9):
        e = _exponent(bound)
        assert bound * 2.0 ** e < 2 ** 14 <= bound * 2.0 ** (e + 1)
        # values across 30 binades below the bound, and the bound itself
        x = (bound * rng.uniform(-1, 1, 200000) * 2.0 ** -rng.integers(0, 30, 200000)).astype(np.float32)
        x[0] = np.float32(bound)
        y = (x * np.float32(2.0 ** e)).astype(np.float32)
        assert np.all(y.astype(np.float64) == x.astype(np.float64) * 2.0 ** e)  # the scaling is exact
        h, m, r = _split(y)
        assert np.all(np.isfinite(h)) and np.abs(h).max() <= 2 ** 14
        assert np.all(r.astype(np.float64) == y.astype(np.float64) - h)  # y - h exact in fp32
        err = np.abs(y.astype(np.float64) - h - m)
        assert np.all(err <= 2.0 ** -22 * np.abs(y) + 2.0 ** -25)
        assert np.all(np.abs(m) <= 2.0 ** -11 * np.abs(y) + 2.0 ** -25)


def test_three_products_and_a_dropped_one(rng):
    a = (rng.standard_normal(100000) * 2.0 ** rng.integers(-8, 8, 100000)).astype(np.float32)
    w = (0.05 * rng.standard_normal(100000)).astype(np.float32)
    ea, ew = _exponent(float(np.abs(a).max())), _exponent(float(np.abs(w).max()))
    ah, am, _ = _split(a * np.float32(2.0 ** ea))
    wh, wm, _ = _split(w * np.float32(2.0 ** ew))
    s = 2.0 ** -(ea + ew)
    exact = a.astype(np.float64) * w
    three = (ah.astype(np.float64) * wh + ah.astype(np.float64) * wm + am.astype(np.float64) * wh) * s
    # relative to |a w| where a is far from the bottom of the scale range
    big = np.abs(a) * 2.0 ** ea > 2.0 ** -3
    rel = np.abs(three - exact)[big] / np.abs(exact)[big]
    assert rel.max() <= 2.0 ** -20
    no_hm = (ah.astype(np.float64) * wh + am.astype(np.float64) * wh) * s
    assert (np.abs(no_hm - exact)[big] / np.abs(exact)[big]).max() > 2.0 ** -14


def test_operand_bounds_hold_and_are_reached(rng):
    D, N = 384, 300
    gamma = (1.0 + 0.4 * rng.standard_normal(D)).astype(np.float32)
    w = (0.05 * rng.standard_normal((N, D))).astype(np.float32)
    b = (0.2 * rng.standard_normal(N)).astype(np.float32)
    x = (rng.standard_normal((3000, D)) * np.exp(2 * rng.standard_normal((3000, 1)))).astype(np.float32)
    x[0] = 0.0
    x[0, np.argmax(np.abs(gamma))] = 3.0  # all mass on the largest gain
    x[1] = np.sign(gamma) * 1e-20         # tiny rows normalise to the same scale
    y = O.rms_norm(x, gamma).astype(np.float64)
    b0 = np.sqrt(D) * np.abs(gamma).max()
    assert np.abs(y).max() <= b0 * (1 + 2.0 ** -20)
    assert np.abs(y[0]).max() >= b0 * (1 - 1e-6)
    z = y @ w.astype(np.float64).T + b
    t = b0 * np.sqrt((w.astype(np.float64) ** 2).sum(1)).max() + np.abs(b).max()
    assert np.abs(z).max() <= t
    g = O.geglu(z[:, : 2 * (N // 2)].astype(np.float32)).astype(np.float64)
    assert np.abs(g).max() <= t * t


def _attention_exponents(bound: float):
    """The fp16 two-piece attention's exponents for a bound B on |q|, |k|,
    |v|: k and q scaled from the rotated bound sqrt(2) B (q also carrying the
    softmax scale 1/8 and log2 e), v from B, the probabilities by 2^5."""
    f32 = np.float32
    qs = f32(0.125) * f32(1.4426950408889634)
    ek = _exponent(float(f32(1.4142135) * f32(1.0001) * f32(bound)))
    eq = _exponent(float(f32(1.4142135) * f32(1.0001) * f32(bound) * qs))
    ev = _exponent(bound)
    return ek, eq, ev


def test_attention_scale_range():
    """Within [2^-40, 2^60] (the range the library runs the fp16 two-piece
    attention on) the single-constant unscales 2^-(ek+eq) and 2^-(ev+5) are
    normal fp32 powers of two; a bound of 1e25 (or 1e-20) takes the scores'
    unscale beyond fp32's exponent range, which is why such bounds run on the
    kernels without piece scales."""
    def normal(e):  # 2^e is a normal, finite fp32
        return -126 <= e <= 127

    for b in np.geomspace(2.0 ** -40, 2.0 ** 60, 997):
        ek, eq, ev = _attention_exponents(float(b))
        assert normal(-(ek + eq)) and normal(-(ev + 5)), b
        assert normal(ek) and normal(eq) and normal(ev)
    ek, eq, _ = _attention_exponents(1.0e25)
    assert -(ek + eq) > 127  # 2^-(ek+eq) overflows to +inf
    ek, eq, _ = _attention_exponents(1.0e-20)
    assert -(ek + eq) < -149  # 2^-(ek+eq) underflows to 0
