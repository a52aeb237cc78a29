"""Pins oracle/p8.py (the int8-activation W4A8 branch) without the reference's tinygrad.

* level table: the 8 IQ3_XXS grid magnitudes map to 1, 3, ..., 15 (rint(v / 4.0507), clipped);
* quantizer: rint is half-even (checked element-wise against Python's round of the float64
  quotient), the extreme element of a chunk lands on +-127, all-zero chunks give 0 with the
  1e-6 floor, every element is within half a step of its value, the row sums are the sums of
  the stored int8s;
* linearized weights: equal to the independent IQ3_XXS lane dequant (oracle.quants) times
  4.0507 * level / magnitude for every element;
* the product: a pure-Python loop on a small case.
"""
import numpy as np

from oracle import p8, quants
from thunderllamax_amd import formats, synth


def test_lut8_levels():
    lut = p8.lut8_ref()
    g = quants._grid_f32().reshape(-1)
    want = {4: 1, 12: 3, 20: 5, 28: 7, 36: 9, 44: 11, 52: 13, 62: 15}
    assert set(np.unique(g).astype(int)) == set(want)
    assert np.array_equal(lut, np.array([want[int(v)] for v in g], dtype=np.int8))


def test_quant_rows_closed_forms():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((5, 512)) * 0.7).astype(np.float16)
    x[1, 128:256] = 0                       # an all-zero chunk
    x[2, 300] = np.float16(-40.0)           # a dominant element
    x[3, 0:128] = np.float16(2.5)           # ties once scaled (many equal values)
    x[3, 7] = np.float16(127.0)
    xq, sx, rs = p8.quant_rows_ref(x)
    xf = x.astype(np.float32)
    for m in range(x.shape[0]):
        for c in range(x.shape[1] // 128):
            seg = xf[m, 128 * c:128 * c + 128]
            am = np.float32(np.abs(seg).max())
            s = np.float32(np.float32(max(am, np.float32(1e-6))) * np.float32(1.0 / 127.0))
            assert sx[m, c] == s
            qs = [max(-127, min(127, round(float(np.float32(v / s))))) for v in seg]   # half-even
            assert np.array_equal(xq[m, 128 * c:128 * c + 128], np.array(qs, dtype=np.int8))
            assert rs[m, c] == sum(qs)
            if am > 0:
                assert np.abs(xq[m, 128 * c:128 * c + 128]).max() == 127
                assert np.all(np.abs(xq[m, 128 * c:128 * c + 128] * np.float64(s) - seg) <= 0.5 * s * (1 + 1e-6))
    assert not xq[1, 128:256].any() and rs[1, 1] == 0 and sx[1, 1] == np.float32(1e-6) * np.float32(1 / 127)
    assert xq[2, 300] == -127


def test_dequant_lin_matches_lane_dequant():
    rng = synth.config_rng(4)
    K = 768
    packed = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, 24, K), K)
    lin = p8.dequant_lin_packed(packed, K).astype(np.float64)
    exact = quants.dequant_iq3xxs_lanes(packed, K).astype(np.float64)
    # the sub-block scale db per weight, from the packed fields directly
    nb = K // 256
    d = np.ascontiguousarray(packed[:, 96 * nb:98 * nb]).view(np.float16).astype(np.float64)
    sw = np.ascontiguousarray(packed[:, 64 * nb:96 * nb]).view("<u4").astype(np.uint64)
    db = d[:, :, None] * (((sw >> 28).astype(np.float64)).reshape(-1, nb, 8) + 0.5) * 0.5
    db = np.repeat(db.reshape(-1, nb * 8), 32, axis=1)
    mag = np.abs(exact) / db
    lev = {4: 1, 12: 3, 20: 5, 28: 7, 36: 9, 44: 11, 52: 13, 62: 15}
    g = np.rint(mag).astype(int)
    assert np.allclose(mag, g, rtol=0, atol=1e-4) and set(np.unique(g)) <= set(lev)
    want = np.sign(exact) * db * float(p8.DELTA) * np.vectorize(lev.get)(g)
    assert np.allclose(lin, want, rtol=2e-6, atol=0)


def test_w4a8_ffn_ref_loop():
    rng = np.random.default_rng(5)
    K = 256
    pg = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, 3, K), K)
    pu = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, 3, K), K)
    wg, wu = p8.dequant_lin_packed(pg, K), p8.dequant_lin_packed(pu, K)
    xq, sx, _ = p8.quant_rows_ref((rng.standard_normal((2, K)) * 0.5).astype(np.float16))
    g, u, out = p8.w4a8_ffn_ref(wg, wu, xq, sx)
    for m in range(2):
        for n in range(3):
            sg = su = 0.0
            for k in range(K):
                xv = int(xq[m, k]) * float(sx[m, k // 128])
                sg += xv * float(wg[n, k])
                su += xv * float(wu[n, k])
            assert abs(sg - g[m, n]) <= 1e-12 * max(1.0, abs(sg))
            assert abs(su - u[m, n]) <= 1e-12 * max(1.0, abs(su))
    assert out.dtype == np.float16 and out.shape == (2, 3)


def test_product_lut8_is_the_oracle_table():
    from thunderllamax_amd import tables
    assert np.array_equal(tables.iq3xxs_lut8(), p8.lut8_ref())
