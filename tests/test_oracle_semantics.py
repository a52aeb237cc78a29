"""Pins oracle.gemv's GEMV / GEMM semantics (the exact product and each kernel's epilogue) by
closed forms on hand-built weights, independently of how the oracle writes them.

Weights are signed, scaled unit rows (row n = c_n * e_{perm(n)}, plus an optional 2^-12 tail
term), so every output is known in closed form; shapes have M != N != K, so a transposed
operand fails on shape or value.  fp16 rounding is checked against Python's own binary16
packing (``struct`` format 'e', round-to-nearest-even), not numpy's cast.

* ``matvec64`` / ``gemv16_ref`` / ``pf_o_ref`` (IQ3ROWP's ``out = half(acc)``,
  /root/reference/engine/aq3k8.cu:125-130; pf_gemm3 :421-423): the half rounding of a sum
  that is not an fp16 number;
* ``down8_ref`` (``y = hh + float(half(acc))``, /root/reference/engine/down8.cu:143): the acc is
  rounded to fp16 before the fp32 residual add;
* ``pf_res_ref`` (``out32 = res + acc``, /root/reference/engine/pf_gemm3.cu:410-414): no half
  rounding;
* ``ffn8_ref`` / ``pf_ffn_ref``: gate and up from their own matrices (a swap changes the value),
  SwiGLU against float64 silu(g) * u;
* ``q6k_gemv_ref``: fp32 x, exact float64 sum;
* ``rel_err``: the norm-wise definition.
"""
import struct

import numpy as np

from oracle import gemv

M, N, K = 3, 5, 7


def _f16(v):
    """Round-to-nearest-even binary16 by Python's struct packing."""
    return struct.unpack("<e", struct.pack("<e", float(v)))[0]


def _unit_rows(rng, tail=0.0):
    perm = rng.permutation(K)[:N]
    c = np.array([1.0, -2.0, 0.5, 4.0, -0.25])
    W = np.zeros((N, K), dtype=np.float32)
    W[np.arange(N), perm] = c
    if tail:
        W[np.arange(N), (perm + 1) % K] = tail
    return W, perm, c


def _x16(rng):
    return rng.integers(-8, 9, size=(M, K)).astype(np.float16) / np.float16(4)


def test_matvec64_is_x_times_w_transposed():
    rng = np.random.default_rng(0)
    W, perm, c = _unit_rows(rng)
    x = _x16(rng)
    got = gemv.matvec64(W, x)
    assert got.shape == (M, N)
    want = x.astype(np.float64)[:, perm] * c[None, :]
    assert np.array_equal(got, want)


def test_half_epilogues_round_a_non_fp16_sum():
    rng = np.random.default_rng(1)
    W, perm, c = _unit_rows(rng, tail=2.0 ** -12)
    x = np.ones((M, K), dtype=np.float16)
    # acc = c_n + 2^-12: not an fp16 number next to 1, 2 and 4 (it rounds to c_n)
    acc_want = c[None, :] + 2.0 ** -12
    for fn in (gemv.gemv16_ref, gemv.pf_o_ref):
        acc, out = fn(W, x)
        assert np.array_equal(acc, np.broadcast_to(acc_want, (M, N)))
        want = np.array([[_f16(v) for v in row] for row in acc_want.repeat(M, 0)])
        assert np.array_equal(out.astype(np.float64), want)
        assert out.dtype == np.float16


def test_down8_rounds_acc_to_half_before_the_residual():
    rng = np.random.default_rng(2)
    W, perm, c = _unit_rows(rng, tail=2.0 ** -12)
    g = np.ones((M, K), dtype=np.float16)
    hh = np.full((M, N), 0.5, dtype=np.float32)
    acc, y = gemv.down8_ref(W, g, hh)
    want = np.float32(0.5) + np.array([_f16(v) for v in c + 2.0 ** -12], dtype=np.float32)
    assert y.dtype == np.float32
    assert np.array_equal(y, np.broadcast_to(want, (M, N)))
    # without the half rounding the sum would keep the 2^-12 term
    assert not np.array_equal(y, (hh + (c + 2.0 ** -12)[None, :]).astype(np.float32))


def test_pf_res_keeps_the_full_fp32_sum():
    rng = np.random.default_rng(3)
    W, perm, c = _unit_rows(rng, tail=2.0 ** -12)
    x = np.ones((M, K), dtype=np.float16)
    res = np.zeros((M, N), dtype=np.float32)
    acc, out = gemv.pf_res_ref(W, x, res)
    want = np.broadcast_to(np.float32(c + 2.0 ** -12), (M, N))
    assert out.dtype == np.float32
    assert np.array_equal(out, want)
    assert not np.array_equal(out, np.float32(c)[None, :].repeat(M, 0))


def test_ffn8_gate_and_up_come_from_their_own_matrices():
    rng = np.random.default_rng(4)
    Wg, pg, cg = _unit_rows(rng)
    Wu, pu, cu = _unit_rows(rng)
    Wu *= 3.0
    x = _x16(rng)
    for fn in (gemv.ffn8_ref, gemv.pf_ffn_ref):
        ag, au, gact = fn(Wg, Wu, x)
        g = x.astype(np.float64)[:, pg] * cg
        u = x.astype(np.float64)[:, pu] * cu * 3.0
        assert np.array_equal(ag, g) and np.array_equal(au, u)
        want = g / (1.0 + np.exp(-g)) * u
        # fp16 chain: within a few fp16 ulps of the float64 SwiGLU
        assert np.all(np.abs(gact.astype(np.float64) - want) <= 4 * 2.0 ** -11 * np.abs(want) + 2.0 ** -24)
        swapped = u / (1.0 + np.exp(-u)) * g
        differs = np.abs(swapped - want) > 8 * 2.0 ** -11 * np.abs(want) + 1e-3
        assert differs.any()


def test_q6k_gemv_ref_fp32_x_exact_sum():
    rng = np.random.default_rng(5)
    W, perm, c = _unit_rows(rng, tail=2.0 ** -30)
    x = rng.standard_normal(K).astype(np.float32)
    y = gemv.q6k_gemv_ref(W, x)
    want = x.astype(np.float64)[perm] * c + x.astype(np.float64)[(perm + 1) % K] * 2.0 ** -30
    assert np.array_equal(y, want)


def test_rel_err_definition():
    ref = np.array([3.0, 4.0])
    assert abs(gemv.rel_err(ref * 1.001, ref) - 1e-3) < 1e-15
    assert abs(gemv.rel_err(ref + np.array([0.0, 0.5]), ref) - 0.1) < 1e-15
    assert gemv.rel_err(ref, ref) == 0.0
