"""RMSNorm activation producers (test infrastructure only): the reference's k0n{M} / hh{M}
(/root/reference/engine/k0n11.cu:88-103, /root/reference/engine/hh11.cu:88-107) in float64.

``rms_ref`` -> the ideal ``x * r * nw`` with ``r = 1 / sqrt(sum(x^2) / D + 1e-6)`` in float64 and
its fp16 rounding; ``add_rms_ref`` adds ``hh = x + float(a)`` in float32 first (an exact IEEE
single-precision add, as the kernels do).  The kernels' fp32 reciprocal square root and
products make their fp16 outputs equal to the rounded ideal or one unit in the last place
away from it.  Pinned by tests/test_oracle_norm.py with closed forms (constant rows, a single
spike, scale invariance).
"""
import numpy as np

EPS = 1e-6


def rms_ref(x, nw):
    """x float32 [M, D], nw float32 [D] -> (ideal float64 [M, D], fp16 [M, D])."""
    x64 = np.asarray(x, dtype=np.float32).astype(np.float64)
    r = 1.0 / np.sqrt((x64 * x64).sum(axis=1) / x64.shape[1] + EPS)
    ideal = x64 * r[:, None] * np.asarray(nw, dtype=np.float32).astype(np.float64)[None, :]
    return ideal, ideal.astype(np.float16)


def add_rms_ref(x, a, nw):
    """-> (hh float32, ideal float64, hhx fp16)."""
    hh = (np.asarray(x, dtype=np.float32) + np.asarray(a, dtype=np.float16).astype(np.float32)).astype(np.float32)
    ideal, h16 = rms_ref(hh, nw)
    return hh, ideal, h16


def within_one_ulp(got16, ideal):
    """Each fp16 value equals the ideal rounded, or is its fp16 neighbour on the ideal's side."""
    got = np.asarray(got16, dtype=np.float16).astype(np.float64)
    r16 = np.asarray(ideal, dtype=np.float64).astype(np.float16)
    up = np.nextafter(r16, np.float16(np.inf)).astype(np.float64)
    dn = np.nextafter(r16, np.float16(-np.inf)).astype(np.float64)
    r = r16.astype(np.float64)
    ideal = np.asarray(ideal, dtype=np.float64)
    side = np.where(ideal > r, up, np.where(ideal < r, dn, r))   # the neighbour toward the ideal
    return (got == r) | (got == side)
