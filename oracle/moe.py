"""Reference semantics of the MoE grouped-expert path (router, sort, grouped GEMMs, combine).

Test infrastructure only (see the package docstring).  Each function restates the reference
at the cited lines; the grouped GEMMs are the exact float64 products of the dequantized
weights (the accuracy contract of the path is rel-err <= 1e-3 against them).
"""
import numpy as np

from . import quants

E = 256          # routed experts
TOPK = 8
HID = 2048       # hidden size
FF = 512         # expert intermediate size
IQ4_ROW_UP = 136 * (HID // 256)      # 1088 B: a gate/up row (k = 2048)
IQ4_ROW_DN = 136 * (FF // 256)       # 272 B: a down row (k = 512)
GATE_BYTES = FF * IQ4_ROW_UP         # 557,056: gate rows, then the up rows (GATE_B4)


def topk_ref(logits):
    """Top-8 of each row and the renormalized softmax over them
    (/root/reference/engine/mm/MM_P1_rt8e256.cu:47-60): 8 masked argmax passes with strict
    ``>`` (ties go to the lower expert id); ``gates[r] = exp(l[sel_r] - max) / sum_r(...)``.
    Returns eids uint16 [P, 8] (rank order) and gates float32 [P, 8]."""
    lg = np.asarray(logits, dtype=np.float32)
    P = lg.shape[0]
    eids = np.empty((P, TOPK), dtype=np.uint16)
    gates = np.empty((P, TOPK), dtype=np.float32)
    for p in range(P):
        l = lg[p].copy()
        m = np.float64(l.max())
        ex = []
        for r in range(TOPK):
            be, bv = 0, l[0]
            for e in range(1, E):
                if l[e] > bv:
                    bv, be = l[e], e
            eids[p, r] = be
            ex.append(np.exp(np.float64(bv) - m))
            l[be] = np.float32(-3.402823466e38)
        gates[p] = (np.array(ex) / np.sum(ex)).astype(np.float32)
    return eids, gates


def route_ref(wrt, wsh, h):
    """rt8e256 (/root/reference/engine/mm/MM_P1_rt8e256.cu:14-61): logits = wrt . h (float64
    here), top-8 + softmax as :func:`topk_ref`, ``sg = 1/(1 + exp(-wsh . h))``."""
    lg64 = np.asarray(h, np.float64) @ np.asarray(wrt, np.float64).T
    eids, gates = topk_ref(lg64.astype(np.float32))
    sg = (1.0 / (1.0 + np.exp(-(np.asarray(h, np.float64) @ np.asarray(wsh, np.float64))))).astype(np.float32)
    return lg64, eids, gates, sg


def sort_ref(eids_flat):
    """mmsort8 (/root/reference/engine/mm/MM_B_mmsort8.cu:35-73): exclusive expert offsets
    eoff[257] and the pair ids sorted by expert, stable in pair order."""
    e = np.asarray(eids_flat, dtype=np.int64).ravel()
    cnt = np.bincount(e, minlength=E)
    eoff = np.zeros(E + 1, dtype=np.int32)
    eoff[1:] = np.cumsum(cnt)
    plist = np.empty(len(e), dtype=np.uint16)
    fill = eoff[:-1].copy()
    for i, ei in enumerate(e):
        plist[fill[ei]] = i
        fill[ei] += 1
    return eoff, plist


def silu64(g):
    g = np.asarray(g, np.float64)
    return g / (1.0 + np.exp(-g))


def up_ref(slab_gate_up, x):
    """One expert's gate+up + SwiGLU (gx8e256up4, /root/reference/engine/mm/MM_P2_gx8e256up4.cu:
    23-53): ``act = silu(Wg . x) * (Wu . x)`` over k = 2048, float64.  slab: u8[2*557056]
    (gate rows then up rows); x [T, 2048] -> act [T, 512]."""
    slab = np.ascontiguousarray(slab_gate_up, dtype=np.uint8)
    Wg = quants.dequant_iq4xs(slab[:GATE_BYTES].reshape(FF, IQ4_ROW_UP), HID)
    Wu = quants.dequant_iq4xs(slab[GATE_BYTES:2 * GATE_BYTES].reshape(FF, IQ4_ROW_UP), HID)
    return swiglu_ref(Wg, Wu, x)


def swiglu_ref(Wg, Wu, x):
    """``silu(Wg . x) * (Wu . x)`` in float64 on dequantized gate / up rows of any weight class
    (the gate+up body every expert kernel shares; up_ref is this on IQ4_XS slabs)."""
    x = np.asarray(x, np.float64)
    return silu64(x @ np.asarray(Wg, np.float64).T) * (x @ np.asarray(Wu, np.float64).T)


def down_ref(slab_down, act):
    """One expert's down projection (gx8e256dn, /root/reference/engine/mm/MM_P2_gx8e256dn.cu:
    9-40): ``part = Wd . act`` over k = 512, float64.  slab: u8[557056]; act [T, 512] ->
    [T, 2048]."""
    Wd = quants.dequant_iq4xs(np.ascontiguousarray(slab_down, dtype=np.uint8).reshape(HID, IQ4_ROW_DN), FF)
    return np.asarray(act, np.float64) @ Wd.astype(np.float64).T


# The checkpoint's classes (the same math on other dequantizers): IQ3_S gate/up slabs of
# 2 x 512 rows x 880 B (gxu_gm / gx8e256up, /root/reference/engine/mm/MM_E_gxu_gm.cu:86-93,
# GATE_B = 450560), Q6_K down slabs of 2048 rows x 420 B (gxm_dn6 / gx8e256dn6,
# /root/reference/engine/mm/MM_B_gxm_dn6.cu:18-25), the Q8_0 shared expert (shexp8,
# /root/reference/engine/mm/MM_P2_shexp8.cu:8-13).
IQ3S_ROW_UP = 8 * quants.IQ3S_BYTES
IQ3S_GATE_BYTES = FF * IQ3S_ROW_UP
Q6K_ROW_DN = 2 * quants.Q6K_BYTES


def up3s_ref(slab_gate_up, grid, x):
    """One IQ3_S expert's gate+up + SwiGLU, float64: x [T, 2048] -> act [T, 512]."""
    slab = np.ascontiguousarray(slab_gate_up, dtype=np.uint8)
    Wg = quants.dequant_iq3s(slab[:IQ3S_GATE_BYTES].reshape(FF, IQ3S_ROW_UP), HID, grid)
    Wu = quants.dequant_iq3s(slab[IQ3S_GATE_BYTES:2 * IQ3S_GATE_BYTES].reshape(FF, IQ3S_ROW_UP), HID, grid)
    return swiglu_ref(Wg, Wu, x)


def down6_ref(slab_down, act):
    """One Q6_K expert's down projection, float64: act [T, 512] -> [T, 2048]."""
    Wd = quants.dequant_q6k(np.ascontiguousarray(slab_down, dtype=np.uint8).reshape(HID, Q6K_ROW_DN), FF)
    return np.asarray(act, np.float64) @ Wd.astype(np.float64).T


def shared8_ref(wg, wu, wd, x):
    """The Q8_0 shared expert over positions x [P, 2048]: ``y = Wd . (silu(Wg . x) * (Wu . x))``,
    float64 -> [P, 2048]."""
    Wg = quants.dequant_q8_0(wg, HID)
    Wu = quants.dequant_q8_0(wu, HID)
    Wd = quants.dequant_q8_0(wd, FF)
    return swiglu_ref(Wg, Wu, x) @ Wd.astype(np.float64).T


def combine_ref(parts, gates, sg, shared, hres):
    """cmbz2048 (/root/reference/engine/mm/MM_P34_cmbz2048.cu:14-28): in ``r`` ascending order,
    then the shared expert, then the residual: ``y = hres + (sum_r g_r * part_r + sg * shared)``
    (float64 here).  parts [P, 8, 2048], gates [P, 8], sg [P], shared/hres [P, 2048]."""
    acc = np.einsum("pr,prk->pk", np.asarray(gates, np.float64), np.asarray(parts, np.float64))
    acc += np.asarray(sg, np.float64)[:, None] * np.asarray(shared, np.float64)
    return np.asarray(hres, np.float64) + acc
