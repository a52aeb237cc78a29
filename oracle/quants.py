"""numpy restatements of the GGUF block dequantizers used on the hot path.

Every function returns float32 values.  Where the reference has several independent
statements of one format (a numpy port and a CUDA kernel's per-lane decode), each is
restated separately so the tests can check them against one another.
"""
import numpy as np

from thunderllamax_amd.tables import IQ3XXS_GRID, KVALUES_IQ4NL

QK = 256                         # weights per superblock
IQ3XXS_BYTES = 98                # d f16 | qs[64] | sw u32[8]
Q6K_BYTES = 210                  # ql[128] | qh[64] | sc i8[16] | d f16
Q6K_PAD_BYTES = 212              # pad[2] | d f16 | sc[16] | ql[128] | qh[64]
IQ4XS_BYTES = 136                # d f16 | scales_h u16 | scales_l[4] | qs[128]
Q4K_BYTES = 144                  # d f16 | dmin f16 | scales[12] | qs[128]
Q5K_BYTES = 176                  # d f16 | dmin f16 | scales[12] | qh[32] | qs[128]
IQ3S_BYTES = 110                 # d f16 | qs[64] | qh[8] | signs[32] | scales[4]
Q80_BYTES = 34                   # d f16 | q i8[32]  (32 weights per block)


def _grid_f32():
    """float32[256, 4] -- grid word bytes, little-endian (/root/reference/engine/pack_w4.py:34)."""
    return IQ3XXS_GRID.astype("<u4").view(np.uint8).reshape(256, 4).astype(np.float32)


def _f16(b):
    """u8[..., 2] -> float32 via fp16 (/root/reference/engine/mm/MM_P0_d2_repack.py:75-76)."""
    return np.ascontiguousarray(b).view(np.float16).astype(np.float32)[..., 0]


def _parity7(v):
    """Parity of the low 7 bits (the even-sign rule, /root/reference/engine/aq3k8.cu:110)."""
    v = v & 0x7F
    p = np.zeros_like(v)
    for i in range(7):
        p ^= (v >> i) & 1
    return p


# --------------------------------------------------------------------------- IQ3_XXS
def dequant_iq3xxs_blocks(blocks):
    """Raw GGUF IQ3_XXS blocks u8[nb, 98] -> float32[nb*256], exact (no fp16 rounding).

    Restates the numpy port of tinygrad's GGUF case 18
    (/root/reference/lineage/a3a/a3a_bench.py:28-39, itself checked bit-exact against the
    fork's ``ggml_data_to_tensor`` there, /root/reference/patches/tinygrad-fork.patch:2075-2087):
    ``db = d*((sw>>28)+0.5)*0.5``; sign byte = ``sidx | parity(sidx)<<7`` with
    ``sidx = (sw >> 7*l) & 0x7F``; ``w = db * grid[qs] * sign``.
    """
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    nb = blocks.shape[0]
    d = _f16(blocks[:, 0:2]).reshape(nb)
    words = np.ascontiguousarray(blocks[:, 66:98]).view("<u4").reshape(nb, 8).astype(np.uint32)
    db = d[:, None] * ((words >> 28).astype(np.float32) + np.float32(0.5)) * np.float32(0.5)
    shifts = np.array([0, 7, 14, 21], dtype=np.uint32)
    sidx = ((words[:, :, None] >> shifts) & 0x7F).reshape(nb, 32)
    sbyte = (sidx | (_parity7(sidx) << 7)).astype(np.uint8)
    signbits = (sbyte[:, :, None] >> np.arange(8, dtype=np.uint8)) & 1
    signs = np.where(signbits == 0, 1.0, -1.0).astype(np.float32).reshape(nb, 8, 4, 8)
    vals = _grid_f32()[blocks[:, 2:66]].reshape(nb, 8, 4, 8)
    return (db[:, :, None, None].astype(np.float32) * vals * signs).reshape(nb * QK)


def dequant_iq3xxs_packed(rows, kdim):
    """Packed IQ3_XXS rows u8[N, 98*NB] -> float32[N, kdim], rounded through fp16.

    Restates ``dequant_iq3xxs`` of /root/reference/engine/pack_w4.py:39-68 (the values the
    engine consumes: dq_iq3_r incl. the fp16 rounding of the dequant product).  Packed row
    layout (/root/reference/engine/pack_w1c.py:18-31): ``[qs 64*NB][sw 32*NB][d 2*NB]``.
    """
    rows = np.ascontiguousarray(rows, dtype=np.uint8)
    n = rows.shape[0]
    nb = kdim >> 8
    assert rows.shape[1] == IQ3XXS_BYTES * nb, rows.shape
    row16 = rows.view("<u2")
    q = row16[:, :nb * 32]
    scp = np.ascontiguousarray(rows[:, 64 * nb:96 * nb]).view("<u4")
    d = np.ascontiguousarray(row16[:, nb * 48:nb * 49]).view(np.float16).astype(np.float32)
    G = _grid_f32()
    W = np.empty((n, nb, 32, 8), dtype=np.float32)
    for lc in range(32):
        cc = lc & 3
        qv = q[:, lc::32].astype(np.uint32)
        swv = scp[:, (lc >> 2)::8].astype(np.uint32)
        db = d * ((swv >> 28).astype(np.float32) + np.float32(0.5)) * np.float32(0.5)
        sidx = (swv >> (7 * cc)) & 0x7F
        spar = _parity7(sidx)
        g0 = G[(qv & 0xFF).astype(np.int64)]
        g1 = G[(qv >> 8).astype(np.int64)]
        sg = np.empty((n, nb, 8), dtype=np.float32)
        for b in range(7):
            sg[:, :, b] = np.where((sidx >> b) & 1, -1.0, 1.0)
        sg[:, :, 7] = np.where(spar != 0, -1.0, 1.0)
        W[:, :, lc, :] = db[..., None] * np.concatenate([g0, g1], axis=2) * sg
    return W.reshape(n, nb * QK).astype(np.float16).astype(np.float32)


def dequant_iq3xxs_lanes(rows, kdim):
    """Packed IQ3_XXS rows -> float32[N, kdim] (fp32, unrounded), via the CUDA per-lane form.

    Restates the ``IQ3ROWP`` body of /root/reference/engine/aq3k8.cu:99-124 element by
    element: lane ``l`` of block ``b`` owns weights ``k = 256*b + 8*l + j``; it reads qs u16
    ``32*b + l``, scale word ``8*b + (l>>2)``, sign field ``l & 3`` and d ``b``.  Written as
    explicit per-lane loops so it shares no indexing code with the vectorized forms above.
    """
    rows = np.ascontiguousarray(rows, dtype=np.uint8)
    n = rows.shape[0]
    nb = kdim >> 8
    G = _grid_f32()
    out = np.empty((n, kdim), dtype=np.float32)
    for r in range(n):
        rowp = rows[r]
        qsp = rowp[:64 * nb].view("<u2")
        scp = rowp[64 * nb:96 * nb].view("<u4")
        dpp = rowp[96 * nb:98 * nb].view(np.float16)
        for b in range(nb):
            d = np.float32(dpp[b])
            for lane in range(32):
                sw = int(scp[8 * b + (lane >> 2)])
                db = np.float32(d * (np.float32(sw >> 28) + np.float32(0.5)) * np.float32(0.5))
                sidx = (sw >> (7 * (lane & 3))) & 0x7F
                spar = bin(sidx).count("1") & 1
                q = int(qsp[32 * b + lane])
                g = list(G[q & 0xFF]) + list(G[q >> 8])
                for j in range(8):
                    neg = ((sidx >> j) & 1) if j < 7 else spar
                    out[r, 256 * b + 8 * lane + j] = db * np.float32(g[j]) * np.float32(-1.0 if neg else 1.0)
    return out


# --------------------------------------------------------------------------- Q6_K
def dequant_q6k(raw, kdim):
    """Raw Q6_K rows u8[N, 210*NB] -> float32[N, kdim].

    Restates ``dq_q6_k`` of /root/reference/engine/mm/MM_P2_ports.py:21-45 (llama.cpp's
    ``dequantize_row_q6_K``): element ``k = 128h + 32g + l``,
    ``q = ((ql[64h+l+32(g&1)] >> 4(g>=2)) & 0xF) | (((qh[32h+l] >> 2g) & 3) << 4)``,
    ``w = (d*sc[8h + l//16 + 2g]) * (q-32)`` in that fp32 order.
    """
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    n = raw.shape[0]
    nb = kdim >> 8
    assert raw.shape[1] == Q6K_BYTES * nb, raw.shape
    blk = raw.reshape(n, nb, Q6K_BYTES)
    ql = blk[:, :, 0:128].astype(np.int32)
    qh = blk[:, :, 128:192].astype(np.int32)
    sc = blk[:, :, 192:208].view(np.int8).astype(np.float32)
    d = _f16(blk[:, :, 208:210])
    y = np.empty((n, nb, QK), dtype=np.float32)
    for h in range(2):
        for l in range(32):
            is_ = l >> 4
            lo_a = ql[:, :, 64 * h + l]
            lo_b = ql[:, :, 64 * h + l + 32]
            hb = qh[:, :, 32 * h + l]
            qs = ((lo_a & 0xF) | ((hb & 3) << 4),
                  (lo_b & 0xF) | (((hb >> 2) & 3) << 4),
                  (lo_a >> 4) | (((hb >> 4) & 3) << 4),
                  (lo_b >> 4) | (((hb >> 6) & 3) << 4))
            for g in range(4):
                t = d * sc[:, :, 8 * h + is_ + 2 * g]
                y[:, :, 128 * h + 32 * g + l] = t * (qs[g] - 32).astype(np.float32)
    return y.reshape(n, kdim)


def dequant_q6k_h6k_lanes(raw, kdim):
    """Raw Q6_K rows -> float32[N, kdim] via the per-lane form of ``h6k2048``.

    Restates /root/reference/engine/mm/MM_P34_h6k2048.cu:18-45: lane ``l`` of half ``hh``
    owns elements ``b*256 + hh*128 + l + {0, 32, 64, 96}``; scale index ``8*hh + (l>>4) +
    {0,2,4,6}``; ``(d*sc) * (int(q) - 32)``.
    """
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    n = raw.shape[0]
    nb = kdim >> 8
    out = np.empty((n, kdim), dtype=np.float32)
    for r in range(n):
        for b in range(nb):
            blk = raw[r, b * Q6K_BYTES:(b + 1) * Q6K_BYTES]
            d = np.float32(blk[208:210].view(np.float16)[0])
            sc = blk[192:208].view(np.int8)
            for lane in range(32):
                is_ = lane >> 4
                for hh in range(2):
                    qb, hb, sb = 64 * hh + lane, 128 + 32 * hh + lane, 8 * hh + is_
                    qhb = int(blk[hb])
                    ql0, ql32 = int(blk[qb]), int(blk[qb + 32])
                    vals = ((ql0 & 0xF) | ((qhb & 3) << 4),
                            (ql32 & 0xF) | (((qhb >> 2) & 3) << 4),
                            (ql0 >> 4) | (((qhb >> 4) & 3) << 4),
                            (ql32 >> 4) | (((qhb >> 6) & 3) << 4))
                    for jj in range(4):
                        t = np.float32(d * np.float32(sc[sb + 2 * jj]))
                        out[r, (b << 8) + (hh << 7) + lane + 32 * jj] = np.float32(t * np.float32(vals[jj] - 32))
    return out


def dequant_q6k_padded_lanes(padded, kdim):
    """Padded Q6_K rows u8[N, 212*NB] -> float32[N, kdim] via the per-lane form of ``aq6k8``.

    Restates /root/reference/engine/aq6k8.cu:141-160 on the 212-byte padded block
    ``[pad2][d2][sc16][lo128][qh64]`` (/root/reference/engine/pack_w1c.py:33-45): lane ``l``
    owns ``k = 256*b + 8*l + j``; lo byte ``20 + 64*(l>>4) + 8*(l&7) + j`` (high nibble when
    ``(l&15) >= 8``); qh byte ``148 + 32*(l>>4) + 8*(l&3) + j`` shifted by ``2*((l>>2)&3)``;
    scale ``sc[l>>1]``.
    """
    padded = np.ascontiguousarray(padded, dtype=np.uint8)
    n = padded.shape[0]
    nb = kdim >> 8
    out = np.empty((n, kdim), dtype=np.float32)
    for r in range(n):
        for b in range(nb):
            blk = padded[r, b * Q6K_PAD_BYTES:(b + 1) * Q6K_PAD_BYTES]
            d = np.float32(blk[2:4].view(np.float16)[0])
            for lane in range(32):
                nib_hi = (lane & 15) >= 8
                c2 = (lane >> 2) & 3
                sc8 = int(blk[4 + (lane >> 1)].view(np.int8))
                for j in range(8):
                    lob = int(blk[20 + 64 * (lane >> 4) + (lane & 7) * 8 + j])
                    xl = (lob >> 4) & 0xF if nib_hi else lob & 0xF
                    qhb = int(blk[148 + (lane >> 4) * 32 + (lane & 3) * 8 + j])
                    xh2 = ((qhb >> (c2 << 1)) & 3) << 4
                    q = (xl | xh2) - 32
                    out[r, (b << 8) + (lane << 3) + j] = np.float32(np.float32(d * np.float32(sc8)) * np.float32(q))
    return out


# --------------------------------------------------------------------------- IQ4_XS
def dequant_iq4xs(raw, kdim):
    """Raw IQ4_XS rows u8[N, 136*NB] -> float32[N, kdim].

    Restates ``dq_iq4_xs`` of /root/reference/engine/mm/MM_P0_d2_repack.py:78-93 (llama.cpp's
    ``dequantize_row_iq4_xs``): group ``ib`` (32 weights) scale
    ``ls = ((sl[ib/2] >> 4(ib&1)) & 0xF) | (((sh >> 2ib) & 3) << 4)``, ``dl = d*(ls-32)``;
    ``y[32ib+j] = dl*kv[qs[16ib+j] & 0xF]``, ``y[32ib+16+j] = dl*kv[qs[16ib+j] >> 4]``.
    """
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    n = raw.shape[0]
    nb = kdim >> 8
    assert raw.shape[1] == IQ4XS_BYTES * nb, raw.shape
    blk = raw.reshape(n, nb, IQ4XS_BYTES)
    d = _f16(blk[:, :, 0:2])
    sh = np.ascontiguousarray(blk[:, :, 2:4]).view("<u2")[:, :, 0].astype(np.int64)
    sl = blk[:, :, 4:8].astype(np.int64)
    qs = blk[:, :, 8:136].reshape(n, nb, 8, 16)
    ib = np.arange(8)
    ls = ((sl[:, :, ib >> 1] >> (4 * (ib & 1))) & 0xF) | (((sh[:, :, None] >> (2 * ib)) & 3) << 4)
    dl = d[:, :, None] * (ls - 32).astype(np.float32)
    T = KVALUES_IQ4NL.astype(np.float32)
    y = np.empty((n, nb, 8, 32), dtype=np.float32)
    y[:, :, :, 0:16] = dl[:, :, :, None] * T[qs & 0xF]
    y[:, :, :, 16:32] = dl[:, :, :, None] * T[qs >> 4]
    return y.reshape(n, kdim)


def dequant_iq4xs_lanes(raw, kdim):
    """Raw IQ4_XS rows -> float32[N, kdim] via the per-lane form of ``gx8e256up4``/``gxm_up4``.

    Restates /root/reference/engine/mm/MM_B_gxm_up4.cu:42-55: lane ``l`` of block ``b``
    owns element ``b*256 + ib*32 + l`` for ``ib`` in 0..7; it reads byte
    ``8 + 16*ib + (8 + (l & 15)) - 8`` (``blk[16*ib + nby]`` with ``nby = 8 + (l&15)``),
    taking the high nibble when ``l & 16``; ``dl = d * (ls - 32)``; ``w = dl * kv[nib]``.
    """
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    n = raw.shape[0]
    nb = kdim >> 8
    kv = KVALUES_IQ4NL.astype(np.float32)
    out = np.empty((n, kdim), dtype=np.float32)
    for r in range(n):
        for b in range(nb):
            blk = raw[r, b * IQ4XS_BYTES:(b + 1) * IQ4XS_BYTES]
            d = np.float32(blk[0:2].view(np.float16)[0])
            sh = int(blk[2:4].view("<u2")[0])
            sl = int(blk[4:8].view("<u4")[0])
            for lane in range(32):
                nby = 8 + (lane & 15)
                for ibb in range(8):
                    byte = int(blk[16 * ibb + nby])
                    nib = (byte >> 4) if (lane & 16) else (byte & 0xF)
                    ls = ((sl >> (8 * (ibb >> 1) + 4 * (ibb & 1))) & 0xF) | (((sh >> (2 * ibb)) & 3) << 4)
                    dl = np.float32(d * np.float32(ls - 32))
                    out[r, b * 256 + ibb * 32 + lane] = np.float32(dl * kv[nib])
    return out


# --------------------------------------------------------------------------- Q4_K / Q5_K
# The reference has no numpy statement of these two formats; its CUDA row bodies define them
# (Q5ROW, /root/reference/engine/head8.cu:65-96; KVBODY8's Q4_K v rows,
# /root/reference/engine/aq3k8.cu:27-61; the index law in /root/reference/docs/DEXT_LAWS.md:
# 190-192).  Both follow ggml's ``dequantize_row_q4_K`` / ``dequantize_row_q5_K`` (the GGUF
# format definition, reached by the reference through tinygrad's ggml bindings):
# ``y = (d*sc)*q - (dmin*m)`` in fp32, no fused multiply-add.  Each format is restated twice:
# in ggml's loop form and in the reference kernels' per-lane form.

def k4_scale_min(sc12):
    """6-bit (scale, min) pairs of the 8 sub-blocks from the 12 packed bytes
    (ggml ``get_scale_min_k4``): j < 4 -> (q[j] & 63, q[j+4] & 63); j >= 4 ->
    ((q[j+4] & 0xF) | (q[j-4] >> 6) << 4, (q[j+4] >> 4) | (q[j] >> 6) << 4)."""
    q = np.asarray(sc12, dtype=np.int64)
    sc = np.empty(q.shape[:-1] + (8,), dtype=np.int64)
    mn = np.empty_like(sc)
    for j in range(8):
        if j < 4:
            sc[..., j] = q[..., j] & 63
            mn[..., j] = q[..., j + 4] & 63
        else:
            sc[..., j] = (q[..., j + 4] & 0xF) | ((q[..., j - 4] >> 6) << 4)
            mn[..., j] = (q[..., j + 4] >> 4) | ((q[..., j] >> 6) << 4)
    return sc, mn


def _kq_dequant_loop(raw, kdim, five):
    nbytes = Q5K_BYTES if five else Q4K_BYTES
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    n = raw.shape[0]
    nb = kdim >> 8
    assert raw.shape[1] == nbytes * nb, raw.shape
    blk = raw.reshape(n, nb, nbytes)
    d = _f16(blk[:, :, 0:2])
    dmin = _f16(blk[:, :, 2:4])
    sc, mn = k4_scale_min(blk[:, :, 4:16])
    qh = blk[:, :, 16:48].astype(np.int64) if five else None
    qs = blk[:, :, 48:176].astype(np.int64) if five else blk[:, :, 16:144].astype(np.int64)
    y = np.empty((n, nb, QK), dtype=np.float32)
    for j in range(4):  # 64 elements per step: low nibbles (sub-block 2j), then high (2j+1)
        for half in range(2):
            s_ = 2 * j + half
            d1 = d * sc[:, :, s_].astype(np.float32)
            m1 = dmin * mn[:, :, s_].astype(np.float32)
            q = (qs[:, :, 32 * j:32 * j + 32] >> (4 * half)) & 0xF
            if five:
                q = q + (((qh >> s_) & 1) << 4)
            y[:, :, 64 * j + 32 * half:64 * j + 32 * half + 32] = (
                d1[:, :, None] * q.astype(np.float32) - m1[:, :, None])
    return y.reshape(n, kdim)


def dequant_q4k(raw, kdim):
    """GGUF Q4_K rows u8[N, 144*NB] -> float32[N, kdim] (ggml loop form)."""
    return _kq_dequant_loop(raw, kdim, False)


def dequant_q5k(raw, kdim):
    """GGUF Q5_K rows u8[N, 176*NB] -> float32[N, kdim] (ggml loop form)."""
    return _kq_dequant_loop(raw, kdim, True)


def _kq_dequant_lanes(raw, kdim, five):
    nbytes = Q5K_BYTES if five else Q4K_BYTES
    qoff = 48 if five else 16
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    n = raw.shape[0]
    nb = kdim >> 8
    out = np.empty((n, kdim), dtype=np.float32)
    for r in range(n):
        for b in range(nb):
            blk = raw[r, b * nbytes:(b + 1) * nbytes].astype(np.int64)
            d = np.float32(raw[r, b * nbytes:b * nbytes + 2].view(np.float16)[0])
            dm = np.float32(raw[r, b * nbytes + 2:b * nbytes + 4].view(np.float16)[0])
            for lane in range(32):
                s_ = lane >> 2
                if s_ < 4:
                    sc, mn = blk[4 + s_] & 63, blk[8 + s_] & 63
                else:
                    sc = (blk[8 + s_] & 0xF) | ((blk[s_] >> 6) << 4)
                    mn = (blk[8 + s_] >> 4) | ((blk[s_ + 4] >> 6) << 4)
                nsh = ((lane >> 2) & 1) * 4
                for j in range(8):
                    qv = (int(blk[qoff + ((lane >> 3) << 5) + ((lane & 3) << 3) + j]) >> nsh) & 0xF
                    if five:
                        qv += ((int(blk[16 + ((lane & 3) << 3) + j]) >> s_) & 1) << 4
                    t = np.float32(d * np.float32(sc))
                    out[r, 256 * b + 8 * lane + j] = np.float32(t * np.float32(qv)) - np.float32(dm * np.float32(mn))
    return out


def dequant_q4k_lanes(raw, kdim):
    """Q4_K rows -> float32 via the per-lane form of KVBODY8 (/root/reference/engine/aq3k8.cu:
    36-55): lane l owns k = 8l + j; qs byte 16 + 32(l>>3) + 8(l&3) + j, nibble 4((l>>2)&1);
    sub-block l>>2 for the 6-bit scale and min."""
    return _kq_dequant_lanes(raw, kdim, False)


def dequant_q5k_lanes(raw, kdim):
    """Q5_K rows -> float32 via the per-lane form of Q5ROW (/root/reference/engine/head8.cu:
    68-90): as Q4_K with qs at byte 48, plus bit (l>>2) of qh byte 16 + 8(l&3) + j as q's bit 4."""
    return _kq_dequant_lanes(raw, kdim, True)


# --------------------------------------------------------------------------- IQ3_S
# The MoE checkpoint's routed gate/up class.  Its 512-entry grid is a third-party table (ggml's
# iq3s_grid, which the reference reaches through tinygrad's ggml bindings and passes to its
# kernels at run time as gridf float[512][4]); it is absent here, so every function takes the
# grid as an argument and the tests run on synthetic grids.
def dequant_iq3s(raw, kdim, grid):
    """IQ3_S rows u8[N, 110*NB] -> float32[N, kdim], grid float32[512, 4].

    Restates ``dq_iq3_s`` of /root/reference/engine/mm/MM_P0_d2_repack.py:95-120: sub-block pair
    ``p`` has ``db1 = d*(1 + 2*(sc[p] & 0xF))``, ``db2 = d*(1 + 2*(sc[p] >> 4))``; half ``h`` of it
    (sub-block 2p+h, 32 weights) reads index bytes ``qs[16p + 8h ..]``, high-bit byte
    ``qh[2p+h]`` and sign bytes ``signs[8p + 4h ..]``; group ``l`` (8 weights) takes indices
    ``ia = qs[2l] | ((qh << (8-2l)) & 256)``, ``ib = qs[2l+1] | ((qh << (7-2l)) & 256)`` and
    ``y = db * grid[ia] | db * grid[ib]``, negated where bit j of ``signs[l]`` is set.
    """
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    G = np.asarray(grid, np.float32).reshape(512, 4)
    n = raw.shape[0]
    nb = kdim >> 8
    assert raw.shape[1] == IQ3S_BYTES * nb, raw.shape
    blk = raw.reshape(n, nb, IQ3S_BYTES)
    d = _f16(blk[:, :, 0:2])
    qs, qh, signs, sc = blk[:, :, 2:66], blk[:, :, 66:74], blk[:, :, 74:106], blk[:, :, 106:110]
    km = (1 << np.arange(8)).astype(np.uint8)
    y = np.empty((n, nb, 8, 32), dtype=np.float32)
    l = np.arange(4)
    for p in range(4):
        for h in range(2):
            db = d * (1 + 2 * ((sc[:, :, p] >> (4 * h)) & 0xF)).astype(np.float32)
            hb = qh[:, :, 2 * p + h].astype(np.int64)
            q = qs[:, :, 16 * p + 8 * h:16 * p + 8 * h + 8].astype(np.int64)
            sg = signs[:, :, 8 * p + 4 * h:8 * p + 4 * h + 4]
            ia = q[:, :, 0:8:2] | ((hb[:, :, None] << (8 - 2 * l)) & 256)
            ib = q[:, :, 1:8:2] | ((hb[:, :, None] << (7 - 2 * l)) & 256)
            neg = (sg[:, :, :, None] & km[None, None, None, :]) != 0
            sgn = np.where(neg, np.float32(-1.0), np.float32(1.0))
            yy = np.empty((n, nb, 4, 8), dtype=np.float32)
            yy[:, :, :, 0:4] = db[:, :, None, None] * G[ia] * sgn[:, :, :, 0:4]
            yy[:, :, :, 4:8] = db[:, :, None, None] * G[ib] * sgn[:, :, :, 4:8]
            y[:, :, 2 * p + h] = yy.reshape(n, nb, 32)
    return y.reshape(n, kdim)


def dequant_iq3s_lanes(raw, kdim, grid):
    """IQ3_S rows -> float32 via the per-weight form of ``gxu_gm``'s tile staging
    (/root/reference/engine/mm/MM_E_gxu_gm.cu:57-84): weight k of a block (kib = k & 255) uses
    index byte ``g = kib >> 2``: ``qb = qs[g] + (((qh[g >> 3] >> (g & 7)) & 1) << 8)``, grid entry
    ``grid[qb][kib & 3]``, scale nibble ``(sc[kib >> 6] >> 4((kib >> 5) & 1)) & 0xF`` as
    ``ds = d * (1 + 2*nib)``, and sign bit ``kib & 7`` of ``signs[kib >> 3]``: ``w = +-ds * g``."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    G = np.asarray(grid, np.float32).reshape(512, 4)
    n = raw.shape[0]
    nb = kdim >> 8
    out = np.empty((n, kdim), dtype=np.float32)
    for r in range(n):
        for b in range(nb):
            blk = raw[r, b * IQ3S_BYTES:(b + 1) * IQ3S_BYTES]
            d = np.float32(blk[0:2].view(np.float16)[0])
            for kib in range(256):
                g = kib >> 2
                qb = int(blk[2 + g]) + (((int(blk[66 + (g >> 3)]) >> (g & 7)) & 1) << 8)
                s_ = kib >> 5
                nib = (int(blk[106 + (s_ >> 1)]) >> (4 * (s_ & 1))) & 0xF
                ds = np.float32(d * np.float32(1.0 + 2.0 * nib))
                w = np.float32(ds * G[qb, kib & 3])
                if (int(blk[74 + (kib >> 3)]) >> (kib & 7)) & 1:
                    w = -w
                out[r, 256 * b + kib] = w
    return out


# --------------------------------------------------------------------------- Q8_0
def dequant_q8_0(raw, kdim):
    """Q8_0 rows u8[N, 34*(kdim/32)] -> float32[N, kdim]: ``y = d * q`` per 32-weight block
    (``dq_q8_0``, /root/reference/engine/mm/MM_P2_ports.py:47-54; the shared expert's class)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    n = raw.shape[0]
    nb = kdim >> 5
    assert raw.shape[1] == Q80_BYTES * nb, raw.shape
    blk = raw.reshape(n, nb, Q80_BYTES)
    d = _f16(blk[:, :, 0:2])
    q = blk[:, :, 2:34].astype(np.int8).astype(np.float32)
    return (d[:, :, None] * q).reshape(n, kdim)
