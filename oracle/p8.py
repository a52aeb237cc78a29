"""numpy restatement of the reference's int8-activation prefill branch (W4A8).

Test infrastructure only: imported by tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline``, never by the product.

* ``quant_rows_ref`` -- the activation quantizer pfk_q8 (/root/reference/engine/pfk_q8.cu:30-59):
  per (row, 128-k chunk) ``s = max(absmax, 1e-6) * (1/127)`` in float32, ``q = rint(x / s)``
  (half-even) clamped to [-127, 127], row sum of the stored int8s.
* ``lut8_ref`` -- the linearized IQ3_XXS codebook (/root/reference/engine/p8_w4ffn7_test.py:44-46):
  ``clip(rint(grid / 4.0507), 0, 15)`` per grid byte.
* ``dequant_lin_packed`` -- the weights the W4A8 kernel multiplies
  (/root/reference/engine/p8_w4ffn7.cu:86-113, restated after its test's ``dq_lin``,
  /root/reference/engine/p8_w4ffn7_test.py:52-80): ``sdb * sign * lut8[g][j]`` with
  ``sdb = d * ((sw >> 28) + 0.5) * 0.5 * 4.0507`` in float32, per 32-weight sub-block.
* ``w4a8_ffn_ref`` -- the product of the dequantized int8 activations ``xq * sx`` and those
  weights in float64, then the pf_gemm3 FFN epilogue ``hmul(hsilu(half(g)), half(u))``
  (/root/reference/engine/p8_w4ffn7.cu:234-255).

Pinned by tests/test_oracle_p8.py against closed forms (levels of the 8 grid magnitudes, the
quantizer's ties / zero chunks / extreme element), against the independent IQ3_XXS lane
dequant of ``oracle.quants`` (the linearized weight is that weight times 4.0507 * level / grid
element by element) and against a pure-Python loop on a small case.
"""
import numpy as np

from oracle import gemv, quants

DELTA = np.float32(4.0507)       # /root/reference/engine/p8_w4ffn7.cu:46
KCH = 128                        # activation quantization chunk (/root/reference/engine/pfk_q8.cu:15)


def quant_rows_ref(x16):
    """fp16 [M, K] -> (xq int8 [M, K], sx float32 [M, K/128], rs int32 [M, K/128])."""
    x = np.asarray(x16, dtype=np.float16).astype(np.float32)
    m, k = x.shape
    assert k % KCH == 0, k
    nch = k // KCH
    seg = x.reshape(m, nch, KCH)
    am = np.abs(seg).max(axis=2)
    s = (np.maximum(am, np.float32(1e-6)) * np.float32(1.0 / 127.0)).astype(np.float32)
    q = np.clip(np.rint(seg / s[:, :, None]), -127, 127).astype(np.int8)
    rs = q.astype(np.int32).sum(axis=2).astype(np.int32)
    return q.reshape(m, k), s, rs


def lut8_ref():
    """int8[1024]: level of grid byte j of grid word g at 4g + j."""
    g = quants._grid_f32().reshape(-1)
    return np.clip(np.rint(g / DELTA), 0, 15).astype(np.int8)


def dequant_lin_packed(rows, kdim, lut8=None):
    """Packed IQ3_XXS rows u8[N, 98*NB] -> float32 [N, kdim] linearized weights."""
    lut = (lut8_ref() if lut8 is None else np.asarray(lut8, dtype=np.int8)).astype(np.float32)
    rows = np.ascontiguousarray(rows, dtype=np.uint8)
    n = rows.shape[0]
    nb = kdim >> 8
    row16 = rows.view("<u2")
    q = row16[:, :nb * 32]
    scp = np.ascontiguousarray(rows[:, 64 * nb:96 * nb]).view("<u4")
    d = np.ascontiguousarray(row16[:, nb * 48:nb * 49]).view(np.float16).astype(np.float32)
    W = np.empty((n, nb, 32, 8), dtype=np.float32)
    for lc in range(32):                       # lane-chunk: 8 weights, k = 8 lc within the block
        cc = lc & 3
        qv = q[:, lc::32].astype(np.uint32)
        swv = scp[:, (lc >> 2)::8].astype(np.uint32)
        sdb = d * ((swv >> 28).astype(np.float32) + np.float32(0.5)) * np.float32(0.5) * DELTA
        sidx = (swv >> (7 * cc)) & 0x7F
        spar = quants._parity7(sidx)
        l0 = lut[((qv & 0xFF) << 2)[..., None] + np.arange(4)]
        l1 = lut[((qv >> 8) << 2)[..., None] + np.arange(4)]
        sg = np.empty((n, nb, 8), dtype=np.float32)
        for b in range(7):
            sg[:, :, b] = np.where((sidx >> b) & 1, -1.0, 1.0)
        sg[:, :, 7] = np.where(spar != 0, -1.0, 1.0)
        W[:, :, lc, :] = sdb[..., None] * (np.concatenate([l0, l1], axis=2) * sg)
    return W.reshape(n, kdim)


def w4a8_ffn_ref(wg_lin, wu_lin, xq, sx):
    """-> (g, u) float64 [M, N] and the fp16 SwiGLU output [M, N]."""
    xq = np.asarray(xq, dtype=np.int8)
    xd = xq.astype(np.float64) * np.repeat(np.asarray(sx, dtype=np.float64), KCH, axis=1)
    g = xd @ np.asarray(wg_lin, dtype=np.float64).T
    u = xd @ np.asarray(wu_lin, dtype=np.float64).T
    return g, u, gemv.swiglu16(g, u)
