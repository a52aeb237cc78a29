"""Pins oracle/norm.py by closed forms of RMSNorm."""
import numpy as np

from oracle import norm


def test_constant_rows():
    D = 512
    nw = np.linspace(0.5, 1.5, D).astype(np.float32)
    for c in (3.0, -0.25, 40.0):
        x = np.full((1, D), c, dtype=np.float32)
        ideal, _ = norm.rms_ref(x, nw)
        want = np.sign(c) * nw.astype(np.float64) * abs(c) / np.sqrt(c * c + 1e-6)
        assert np.allclose(ideal[0], want, rtol=1e-15, atol=0)


def test_single_spike():
    D = 5120
    x = np.zeros((1, D), dtype=np.float32)
    x[0, 17] = 100.0
    nw = np.ones(D, dtype=np.float32)
    ideal, h = norm.rms_ref(x, nw)
    assert abs(ideal[0, 17] - 100.0 / np.sqrt(100.0 ** 2 / D + 1e-6)) < 1e-12 and not ideal[0, :17].any()
    assert abs(ideal[0, 17] - np.sqrt(D)) < 1e-3     # eps is negligible against 100^2 / D


def test_scale_invariance_and_add():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    nw = rng.standard_normal(256).astype(np.float32)
    a, _ = norm.rms_ref(x, nw)
    b, _ = norm.rms_ref(x * np.float32(64.0), nw)   # eps negligible at this scale
    assert np.allclose(a, b, rtol=1e-6)
    att = rng.standard_normal((3, 256)).astype(np.float16)
    hh, ideal, _ = norm.add_rms_ref(x, att, nw)
    assert np.array_equal(hh, x + att.astype(np.float32))
    assert np.allclose(ideal, norm.rms_ref(hh, nw)[0], rtol=0, atol=0)


def test_within_one_ulp_accepts_only_the_ideal_side():
    """The fp16 check the producer tests use: the rounded ideal, or its neighbour on the ideal's
    side (an fp32 chain can cross that midpoint only); the other neighbour and 2 ulps fail."""
    ideal = np.array([1.0 + 0.3 * 2.0 ** -10, 1.0 - 0.3 * 2.0 ** -11, 3.0, -2.0 - 0.4 * 2.0 ** -9])
    r = ideal.astype(np.float16)
    up = np.nextafter(r, np.float16(np.inf))
    dn = np.nextafter(r, np.float16(-np.inf))
    toward = np.where(ideal > r.astype(np.float64), up, dn)
    away = np.where(ideal > r.astype(np.float64), dn, up)
    assert norm.within_one_ulp(r, ideal).all()
    assert list(norm.within_one_ulp(toward, ideal)) == [True, True, False, True]   # 3.0 is exact
    assert not norm.within_one_ulp(away, ideal).any()
    assert not norm.within_one_ulp(np.nextafter(toward, toward + (toward - r)), ideal).any()
