"""Pins oracle.gemv's fp16 SiLU / SwiGLU epilogue chain (/root/reference/engine/ffn8.cu:22-24,184).

``hsilu16(h) = fp16(h * fp16(1 / fp16(1 + fp16(exp2(fp16(h * c))))))`` with c = fp16(-log2 e).
It is checked over every finite fp16 input against the float64 silu ``h / (1 + e^-h)``:

* first-order error bound of the chain (five fp16 roundings, unit roundoff u = 2^-11, plus the
  constant's own relative error gamma = |c - (-log2 e)| / log2 e):
  with t = -h log2 e, w = 2^t / (1 + 2^t) and dt = |t| (gamma + u) + 2^-25 (the last term: the
  absolute rounding of a subnormal t),
      |silu16(h) - silu(h)| <= (w (2^dt (1 + u) - 1) + 3u (1 + 4u)) |silu(h)| + 2^-25;
  the exponent error dt moves 2^t by the factor 2^dt, which moves 1 / (1 + 2^t) by at most w
  times that relative change; the rounded sum, reciprocal and product add u each; 2^-25 is the
  absolute rounding of a subnormal result;
* the exp2 overflow branch (fp16(2^t) = inf, h <= -11.09375): the chain gives -0 exactly;
* the exp2 underflow branch (2^t rounds to 0): silu16(h) = h exactly; silu16(+-0) = +-0;
* planted mistakes (a sign flip of the constant, a dropped "1 +", exp in place of exp2, a
  product in place of the reciprocal) each break the bound somewhere, so the bound is tight
  enough to catch them.

``swiglu16(g, u) = fp16(silu16(g) * fp16(u))`` is pinned by its algebra: u = 0 gives 0, u = 1
gives silu16(g), u -> -u negates, u -> 2u doubles (exact in fp16 away from over/underflow), and
against float64 silu(g) * u within the silu bound plus one rounding.
"""
import numpy as np
import pytest

from oracle.gemv import SILU_C16, hsilu16, swiglu16

U16 = 2.0 ** -11
C_TRUE = -1.0 / np.log(2.0)
GAMMA = abs((float(SILU_C16) - C_TRUE) / C_TRUE)


def _all_finite_f16():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    return h[np.isfinite(h)]


def _silu64(h):
    h = np.asarray(h, dtype=np.float64)
    with np.errstate(over="ignore"):
        return h / (1.0 + np.exp(-h))


def _bound(h):
    """Per-element absolute error bound of the fp16 chain (module docstring)."""
    hd = np.asarray(h, dtype=np.float64)
    t = hd * C_TRUE
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp2(t)
        w = np.where(np.isinf(e), 1.0, e / (1.0 + e))
    dt = np.abs(t) * (GAMMA + U16) + 2.0 ** -25
    rel = w * (np.exp2(dt) * (1 + U16) - 1) + 3 * U16 * (1 + 4 * U16)
    return rel * np.abs(_silu64(hd)) + 2.0 ** -25


def _overflows(h):
    """fp16(exp2(fp16(h * c))) is inf: the reference's chain returns h * 0."""
    h = np.asarray(h, dtype=np.float16)
    with np.errstate(over="ignore"):
        t = (h.astype(np.float32) * np.float32(SILU_C16)).astype(np.float16)
        return ~np.isfinite(np.exp2(t.astype(np.float64)).astype(np.float16))


def _chain(h, c=SILU_C16, one=1.0, base2=True, recip=True):
    """The same five-rounding chain with optional planted mistakes (oracle-side mutants)."""
    h = np.asarray(h, dtype=np.float16)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        t = (h.astype(np.float32) * np.float32(c)).astype(np.float16)
        ex = np.exp2 if base2 else np.exp
        e = ex(t.astype(np.float64)).astype(np.float16)
        den = (np.float32(one) + e.astype(np.float32)).astype(np.float16)
        r = (1.0 / den.astype(np.float64) if recip else den.astype(np.float64)).astype(np.float16)
        return (h.astype(np.float32) * r.astype(np.float32)).astype(np.float16)


def test_hsilu16_all_fp16_within_bound():
    h = _all_finite_f16()
    assert h.size == 63488
    y = hsilu16(h).astype(np.float64)
    ok = ~_overflows(h)
    err = np.abs(y - _silu64(h))
    bad = ok & ~(err <= _bound(h))
    assert not bad.any(), f"{bad.sum()} inputs outside the bound, e.g. h={h[bad][:5]}"
    # the bound is not vacuous: over |h| < 8 it stays under 1% relative
    small = ok & (np.abs(h.astype(np.float64)) < 8) & (np.abs(_silu64(h)) > 1e-3)
    assert (_bound(h)[small] / np.abs(_silu64(h))[small]).max() < 0.01


def test_hsilu16_overflow_branch_is_negative_zero():
    h = _all_finite_f16()
    ovf = _overflows(h)
    assert ovf.any()
    hv = h[ovf].astype(np.float64)
    assert hv.max() == -11.09375 and (hv < 0).all()
    y = hsilu16(h[ovf])
    assert (y == 0).all() and np.signbit(y).all()
    # the true value there is tiny: the branch is where the reference flushes silu to -0
    assert np.abs(_silu64(hv)).max() < 2e-4


def test_hsilu16_underflow_branch_is_identity():
    h = _all_finite_f16()
    hd = h.astype(np.float64)
    big = hd > 18.0                       # 2^(-18 log2 e) = 1.5e-8 rounds to fp16 0
    assert big.sum() > 1000
    assert np.array_equal(hsilu16(h[big]), h[big])
    z = np.array([0.0, -0.0], dtype=np.float16)
    y = hsilu16(z)
    assert (y == 0).all() and not np.signbit(y[0]) and np.signbit(y[1])


@pytest.mark.parametrize("mutant", [
    dict(c=np.float16(1.4423828125)),     # sign of the constant flipped
    dict(one=0.0),                        # "1 +" dropped
    dict(base2=False),                    # exp in place of exp2
    dict(recip=False),                    # den instead of 1 / den
])
def test_hsilu16_bound_catches_planted_mistakes(mutant):
    h = _all_finite_f16()
    h = h[np.abs(h.astype(np.float64)) < 10]
    assert np.array_equal(_chain(h), hsilu16(h)), "the unmutated chain is the oracle"
    y = _chain(h, **mutant).astype(np.float64)
    with np.errstate(invalid="ignore"):
        bad = ~(np.abs(y - _silu64(h)) <= _bound(h))
    assert bad.any()


def _grid():
    rng = np.random.default_rng(7)
    g = np.concatenate([rng.standard_normal(4000) * 4, np.linspace(-12, 20, 2000)]).astype(np.float16)
    u = np.concatenate([rng.standard_normal(4000) * 4, np.linspace(-20, 12, 2000)]).astype(np.float16)
    return g, u


def test_swiglu16_algebra():
    g, u = _grid()
    s = hsilu16(g)
    assert np.array_equal(swiglu16(g, np.zeros_like(u)) == 0, np.ones(g.size, dtype=bool))
    assert np.array_equal(swiglu16(g, np.ones_like(u)), s)
    a, b = swiglu16(g, u), swiglu16(g, -u)
    assert np.array_equal(a.astype(np.float64), -b.astype(np.float64))
    # doubling u doubles the fp16 result exactly where neither over- nor underflows
    a2 = swiglu16(g, (u.astype(np.float32) * 2).astype(np.float16)).astype(np.float64)
    normal = (np.abs(a.astype(np.float64)) > 2.0 ** -13) & (np.abs(a.astype(np.float64)) < 30000)
    assert np.array_equal(a2[normal], 2 * a.astype(np.float64)[normal])
    assert (swiglu16(np.zeros_like(g), u) == 0).all()


def test_swiglu16_vs_float64():
    g, u = _grid()
    ud = u.astype(np.float64)
    y = swiglu16(g, u).astype(np.float64)
    ok = ~_overflows(g)
    ref = _silu64(g) * ud
    tol = _bound(g) * np.abs(ud) + U16 * np.abs(ref) * (1 + 2 * U16) + 2.0 ** -25
    assert (np.abs(y - ref)[ok] <= tol[ok]).all()
