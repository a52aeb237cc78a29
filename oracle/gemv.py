"""Reference semantics of the decode GEMVs (float64 ideal + the reference's fp16 epilogues).

The reference kernels compute ``acc_f32 += f32(f16(x) * f16(w))`` -- fp16-rounded weights
and products, fp32 sums (/root/reference/engine/ffn8.cu:155-184).  The accuracy contract
for matmul outputs is a relative error of at most 1e-3 against the exact product of the
dequantized weights and the fp16 activations; ``*_ref`` below compute that exact product in
float64 and then apply each kernel's output epilogue.
"""
import numpy as np

SILU_C16 = np.float16(-1.4423828125)   # fp16(-log2 e), /root/reference/engine/ffn8.cu:23


def hsilu16(h):
    """fp16 SiLU chain of /root/reference/engine/ffn8.cu:22-24, every step rounded to fp16:
    ``h * rcp(1 + exp2(h * c))``."""
    h = np.asarray(h, dtype=np.float16)
    with np.errstate(over="ignore"):          # h * c or exp2 overflowing fp16 -> inf, as on the GPU
        t = (h.astype(np.float32) * np.float32(SILU_C16)).astype(np.float16)
        e = np.exp2(t.astype(np.float64)).astype(np.float16)
    den = (np.float32(1.0) + e.astype(np.float32)).astype(np.float16)
    r = (1.0 / den.astype(np.float64)).astype(np.float16)
    return (h.astype(np.float32) * r.astype(np.float32)).astype(np.float16)


def swiglu16(ag, au):
    """``gact = hmul(hsilu(half(ag)), half(au))`` (/root/reference/engine/ffn8.cu:184)."""
    s = hsilu16(np.asarray(ag).astype(np.float16))
    return (s.astype(np.float32) * np.asarray(au).astype(np.float16).astype(np.float32)).astype(np.float16)


def matvec64(W, x16):
    """Exact product: W float32 [N, K] (dequantized), x fp16 [M, K] -> float64 [M, N]."""
    return np.asarray(x16, dtype=np.float64) @ np.asarray(W, dtype=np.float64).T


def ffn8_ref(Wg, Wu, x16):
    """ffn8 / ffn8v{M}: -> (ag, au) float64 [M, N] and gact fp16 [M, N]."""
    ag, au = matvec64(Wg, x16), matvec64(Wu, x16)
    return ag, au, swiglu16(ag, au)


def down8_ref(Wd, gact16, hh):
    """down8: ``y = hh + float(half(acc))`` (/root/reference/engine/down8.cu:143) -> (acc, y)."""
    acc = matvec64(Wd, gact16)
    y = (np.asarray(hh, dtype=np.float32) + acc.astype(np.float16).astype(np.float32)).astype(np.float32)
    return acc, y


def gemv16_ref(W, x16):
    """IQ3ROWP segment: ``out = half(acc)`` -> (acc, out fp16)."""
    acc = matvec64(W, x16)
    return acc, acc.astype(np.float16)


def q6k_gemv_ref(W, x32):
    """h6k2048 contract: fp32 W (dequantized) times fp32 x, exact in float64 -> [rows]."""
    return np.asarray(W, dtype=np.float64) @ np.asarray(x32, dtype=np.float64)


def pf_ffn_ref(Wg, Wu, x16):
    """pf_gemm3 FFN=1 epilogue ``hmul(hsilu_h(half(g)), half(u))``
    (/root/reference/engine/pf_gemm3.cu:87-89, :415-420): the ffn8 epilogue on M rows."""
    return ffn8_ref(Wg, Wu, x16)


def pf_res_ref(W, x16, res):
    """pf_gemm3 RES=1 epilogue ``out32 = res16 + acc`` -- fp32, no half rounding of acc
    (/root/reference/engine/pf_gemm3.cu:410-414) -> (acc float64, out float32)."""
    acc = matvec64(W, x16)
    return acc, (np.asarray(res, dtype=np.float64) + acc).astype(np.float32)


def pf_o_ref(W, x16):
    """pf_gemm3 plain epilogue ``out16 = half(acc)`` (/root/reference/engine/pf_gemm3.cu:421-423)."""
    return gemv16_ref(W, x16)


def rel_err(y, ref):
    """Norm-wise relative error ||y - ref|| / ||ref|| (float64)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-300))
