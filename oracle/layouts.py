"""numpy restatements of the reference's weight repackers (pure byte permutations).

* ``pack_iq3_w1c``  -- /root/reference/engine/pack_w1c.py:18-31  raw IQ3_XXS rows -> packed rows
* ``pack_q6_pad``   -- /root/reference/engine/pack_w1c.py:33-45  raw Q6_K rows -> 212-B blocks
* ``pack_w7``       -- /root/reference/engine/pack_w7.py:40-73   packed IQ3 rows -> packed7 units
* ``unpack_w7``     -- /root/reference/engine/pack_w7.py:75-96   the inverse
* ``pack_tiled`` / ``unpack_tiled`` -- this library's tile-major records for the IQ3_XXS
  decode GEMVs (no reference counterpart): a lossless re-encoding of the pack_w1c rows above
  with the per-chunk table indices precomputed.  Pinned by the inverse (which also checks the
  one redundant bit, the sign parity), by a hand-decoded block, and, on the GPU, by the GEMVs
  over the records against the dequantized rows.
* ``pack_iq4_tiled`` / ``unpack_iq4_tiled`` -- this library's tiled IQ4_XS expert slabs for the
  MoE GEMMs (no reference counterpart): a byte permutation of GGUF IQ4_XS rows
  (/root/reference/engine/mm/MM_P0_d2_repack.py:78-93 gives the block: d, scales_h, scales_l,
  qs) into MFMA lane order.  Pinned by the inverse, by hand-placed bytes, and, on the GPU, by
  the GEMMs over tiled slabs equal to those over the GGUF rows bit for bit.
* ``pack_iq3s_tiled`` / ``pack_q6k_tiled`` and their inverses -- this library's tiled IQ3_S /
  Q6_K expert slabs for the checkpoint-class MoE GEMMs (no reference counterpart): byte
  permutations of GGUF IQ3_S rows (/root/reference/engine/mm/MM_P0_d2_repack.py:95-120 gives the
  block: d, qs, qh, signs, scales) and Q6_K rows (ql, qh, scales, d) into lane order.  Pinned by
  the inverses, by hand-placed bytes, and, on the GPU, by every routed form over tiled slabs
  equal to the GGUF-row form bit for bit.
"""
import numpy as np


def pack_iq3_w1c(raw_rows, kdim):
    """u8[N, 98*NB] raw GGUF rows -> u8[N, 98*NB] as ``[qs 64NB][sw 32NB][d 2NB]``."""
    nb = kdim // 256
    x = np.ascontiguousarray(raw_rows, dtype=np.uint8).reshape(-1, nb, 98)
    n = x.shape[0]
    out = np.empty((n, 98 * nb), dtype=np.uint8)
    out[:, :64 * nb] = x[:, :, 2:66].reshape(n, 64 * nb)
    out[:, 64 * nb:96 * nb] = x[:, :, 66:98].reshape(n, 32 * nb)
    out[:, 96 * nb:98 * nb] = x[:, :, 0:2].reshape(n, 2 * nb)
    return out


def unpack_iq3_w1c(packed_rows, kdim):
    """Inverse of :func:`pack_iq3_w1c`."""
    nb = kdim // 256
    p = np.ascontiguousarray(packed_rows, dtype=np.uint8)
    n = p.shape[0]
    x = np.empty((n, nb, 98), dtype=np.uint8)
    x[:, :, 2:66] = p[:, :64 * nb].reshape(n, nb, 64)
    x[:, :, 66:98] = p[:, 64 * nb:96 * nb].reshape(n, nb, 32)
    x[:, :, 0:2] = p[:, 96 * nb:98 * nb].reshape(n, nb, 2)
    return x.reshape(n, 98 * nb)


def pack_q6_pad(raw_rows, kdim):
    """u8[N, 210*NB] raw Q6_K rows -> u8[N, 212*NB] blocks ``[pad2][d2][sc16][lo128][qh64]``."""
    nb = kdim // 256
    x = np.ascontiguousarray(raw_rows, dtype=np.uint8).reshape(-1, nb, 210)
    n = x.shape[0]
    out = np.zeros((n, nb, 212), dtype=np.uint8)
    out[:, :, 2:4] = x[:, :, 208:210]
    out[:, :, 4:20] = x[:, :, 192:208]
    out[:, :, 20:148] = x[:, :, 0:128]
    out[:, :, 148:212] = x[:, :, 128:192]
    return out.reshape(n, 212 * nb)


def pack_w7(packed_rows, kdim):
    """Packed IQ3 rows u8[N, 98*NB] -> packed7 u8[N/8, K/128, 32, 16].

    Unit ``r*4 + c`` of (8-row group, 128-k chunk): q u16 words of lane-chunks
    ``lc0 + 4c + cc`` (cc = 0..3), the scale word ``8b + 4h + c``, the block's d, 2 zero bytes;
    ``b = chunk >> 1``, ``h = chunk & 1``, ``lc0 = 16h``.
    """
    p = np.ascontiguousarray(packed_rows, dtype=np.uint8)
    n = p.shape[0]
    assert n % 8 == 0
    nb = kdim >> 8
    nch = kdim // 128
    row16 = p.view("<u2")
    q = row16[:, :nb * 32]
    sc16 = row16[:, nb * 32:nb * 48]
    dp = row16[:, nb * 48:nb * 49]
    out = np.zeros((n // 8, nch, 32, 8), dtype="<u2")
    for chunk in range(nch):
        b, h = chunk >> 1, chunk & 1
        lc0 = 16 * h
        for c in range(4):
            src = q[:, 32 * b + lc0 + 4 * c:32 * b + lc0 + 4 * c + 4]
            w = 8 * b + 4 * h + c
            for r in range(8):
                out[:, chunk, 4 * r + c, 0:4] = src[r::8]
                out[:, chunk, 4 * r + c, 4] = sc16[r::8, 2 * w]
                out[:, chunk, 4 * r + c, 5] = sc16[r::8, 2 * w + 1]
                out[:, chunk, 4 * r + c, 6] = dp[r::8, b]
    return out.view(np.uint8).reshape(n // 8, nch, 32, 16)


def unpack_w7(p7, kdim, n):
    """Inverse of :func:`pack_w7` -> packed IQ3 rows u8[n, 98*NB]."""
    nb = kdim >> 8
    nch = kdim // 128
    u = np.ascontiguousarray(p7, dtype=np.uint8).view("<u2").reshape(n // 8, nch, 32, 8)
    back = np.zeros((n, 49 * nb), dtype="<u2")
    for chunk in range(nch):
        b, h = chunk >> 1, chunk & 1
        lc0 = 16 * h
        for c in range(4):
            w = 8 * b + 4 * h + c
            for r in range(8):
                back[r::8, 32 * b + lc0 + 4 * c:32 * b + lc0 + 4 * c + 4] = u[:, chunk, 4 * r + c, 0:4]
                back[r::8, nb * 32 + 2 * w] = u[:, chunk, 4 * r + c, 4]
                back[r::8, nb * 32 + 2 * w + 1] = u[:, chunk, 4 * r + c, 5]
                back[r::8, nb * 48 + b] = u[:, chunk, 4 * r + c, 6]
    return back.view(np.uint8).reshape(n, 98 * nb)



def _tiled_fields(full, nb):
    """(qs u8[R, NB, 64], sw u32[R, NB, 8], d u16[R, NB]) of packed rows."""
    r = len(full)
    qs = full[:, :64 * nb].reshape(r, nb, 64)
    sw = np.ascontiguousarray(full[:, 64 * nb:96 * nb]).view("<u4").reshape(r, nb, 8)
    d = np.ascontiguousarray(full[:, 96 * nb:]).view("<u2").reshape(r, nb)
    return qs, sw, d


def pack_tiled(packed_rows, kdim):
    """Packed IQ3 rows u8[N, 98*NB] -> tiled records u8[ceil(N/16), NB, 1632].

    Record (tile t, block b): ``[A: slot 0..63 x 16 B][B: slot 0..63 x 8 B][scale word: row
    0..15 x 4 B][d: row 0..15 x 2 B]``.  Slot ``L = 16*kq + r`` (row ``16t + r``) holds the 24-B
    stream of lane-chunks ``lc = 8kq + c``, c = 0..7, 3 little-endian bytes each:
    ``v = i0 | i1 << 12`` with ``i0 = (sidx & 15) << 8 | qs[2lc]``,
    ``i1 = ((sidx >> 4) | parity(sidx) << 3) << 8 | qs[2lc + 1]`` and
    ``sidx = (sw[lc >> 2] >> 7*(lc & 3)) & 127`` (the GGUF sign field of the chunk); its first 16
    bytes go to A, the last 8 to B.  Scale word: nibble j = ``sw[j] >> 28``.  Rows past N are zero.
    """
    p = np.ascontiguousarray(packed_rows, dtype=np.uint8)
    n, nb = len(p), kdim // 256
    t = -(-n // 16)
    full = np.zeros((16 * t, 98 * nb), dtype=np.uint8)
    full[:n] = p
    qs, sw, d = _tiled_fields(full, nb)
    lc = np.arange(32)
    sidx = (sw[:, :, lc >> 2] >> (7 * (lc & 3)).astype(np.uint32)) & 0x7F          # [R, NB, 32]
    par = np.zeros_like(sidx)
    for k in range(7):
        par ^= (sidx >> k) & 1
    i0 = ((sidx & 0xF) << 8) | qs[:, :, 0::2]
    i1 = (((sidx >> 4) | (par << 3)) << 8) | qs[:, :, 1::2]
    v = (i0 | (i1 << 12)).astype(np.uint32)                                          # 24-bit values
    stream = np.stack([v & 0xFF, (v >> 8) & 0xFF, (v >> 16) & 0xFF], axis=-1).astype(np.uint8)
    stream = stream.reshape(t, 16, nb, 4, 24)                                        # [tile, r, b, kq, 24 B]
    A = stream[..., :16].transpose(0, 2, 3, 1, 4).reshape(t, nb, 1024)             # slot = 16kq + r
    B = stream[..., 16:].transpose(0, 2, 3, 1, 4).reshape(t, nb, 512)
    scw = np.zeros(sw.shape[:2], dtype=np.uint32)
    for j in range(8):
        scw |= (sw[:, :, j] >> 28) << (4 * j)
    S = scw.astype("<u4").view(np.uint8).reshape(t, 16, nb, 4).transpose(0, 2, 1, 3).reshape(t, nb, 64)
    D = d.astype("<u2").view(np.uint8).reshape(t, 16, nb, 2).transpose(0, 2, 1, 3).reshape(t, nb, 32)
    return np.ascontiguousarray(np.concatenate([A, B, S, D], axis=2))


def unpack_tiled(rec, kdim, n):
    """Inverse of :func:`pack_tiled` -> packed IQ3 rows u8[n, 98*NB].  Raises if a stored parity
    bit disagrees with its sign field (the one redundant bit of the record)."""
    nb = kdim // 256
    r = np.ascontiguousarray(rec, dtype=np.uint8).reshape(-1, nb, 1632)
    t = len(r)
    A = r[:, :, :1024].reshape(t, nb, 4, 16, 16)
    B = r[:, :, 1024:1536].reshape(t, nb, 4, 16, 8)
    stream = np.concatenate([A, B], axis=-1).transpose(0, 3, 1, 2, 4)               # [tile, r, b, kq, 24]
    b3 = stream.reshape(16 * t, nb, 32, 3).astype(np.uint32)                        # lc = 8kq + c
    v = b3[..., 0] | (b3[..., 1] << 8) | (b3[..., 2] << 16)
    i0, i1 = v & 0xFFF, v >> 12
    sidx = (i0 >> 8) | ((i1 >> 8) & 7) << 4
    par = np.zeros_like(sidx)
    for k in range(7):
        par ^= (sidx >> k) & 1
    if np.any(((i1 >> 11) & 1) != par):
        raise ValueError("tiled record: parity bit does not match its sign field")
    qs = np.empty((16 * t, nb, 64), dtype=np.uint8)
    qs[:, :, 0::2] = i0 & 0xFF
    qs[:, :, 1::2] = i1 & 0xFF
    scw = r[:, :, 1536:1600].reshape(t, nb, 16, 4).transpose(0, 2, 1, 3).reshape(16 * t, nb, 4)
    scw = np.ascontiguousarray(scw).view("<u4")[..., 0]
    sw = np.zeros((16 * t, nb, 8), dtype=np.uint32)
    for j in range(8):
        w = (scw >> (4 * j)) & 0xF
        sw[:, :, j] = w << 28
        for f in range(4):
            sw[:, :, j] |= sidx[:, :, 4 * j + f] << (7 * f)
    d = r[:, :, 1600:].reshape(t, nb, 16, 2).transpose(0, 2, 1, 3).reshape(16 * t, nb, 2)
    out = np.concatenate([qs.reshape(16 * t, 64 * nb),
                          sw.astype("<u4").view(np.uint8).reshape(16 * t, 32 * nb),
                          np.ascontiguousarray(d).reshape(16 * t, 2 * nb)], axis=1)
    return out[:n]


def pack_iq4_tiled(raw_rows, kdim):
    """GGUF IQ4_XS rows u8[N, 136*NB] (N % 16 == 0) -> tiled records u8[N/16, NB, 2176].

    Record (tile t, block b): ``[row r's 8-B header (d, scales_h, scales_l), r = 0..15]`` then two
    1024-B lane regions; lane ``l = 16*kq + r`` of region h holds row ``16t + r``'s quant bytes
    ``qs[64h + 16kq .. 64h + 16kq + 15]`` (sub-block ``4h + kq``; ``qs`` = block bytes 8..135).
    """
    x = np.ascontiguousarray(raw_rows, dtype=np.uint8)
    n, nb = len(x), kdim // 256
    assert n % 16 == 0 and x.shape[1] == 136 * nb
    blk = x.reshape(n // 16, 16, nb, 136).transpose(0, 2, 1, 3)                     # [t, b, r, 136]
    hdr = blk[..., :8].reshape(n // 16, nb, 128)
    lanes = blk[..., 8:].reshape(n // 16, nb, 16, 2, 4, 16).transpose(0, 1, 3, 4, 2, 5)   # [t, b, h, kq, r, 16]
    return np.ascontiguousarray(np.concatenate([hdr, lanes.reshape(n // 16, nb, 2048)], axis=2))


def unpack_iq4_tiled(rec, kdim):
    """Inverse of :func:`pack_iq4_tiled` -> GGUF IQ4_XS rows u8[16*T, 136*NB]."""
    nb = kdim // 256
    r = np.ascontiguousarray(rec, dtype=np.uint8).reshape(-1, nb, 2176)
    t = len(r)
    hdr = r[:, :, :128].reshape(t, nb, 16, 8)
    qs = r[:, :, 128:].reshape(t, nb, 2, 4, 16, 16).transpose(0, 1, 4, 2, 3, 5).reshape(t, nb, 16, 128)
    blk = np.concatenate([hdr, qs], axis=3).transpose(0, 2, 1, 3)                   # [t, r, b, 136]
    return np.ascontiguousarray(blk.reshape(16 * t, 136 * nb))


# Tiled checkpoint-class slabs (this library's decode layout for the MoE checkpoint classes): per
# 16-row tile and 256-weight block, the bytes each lane (col, kq) of a wave fetches for its 64
# weights of the block, in lane order (lane l = 16 kq + col), so every wave load is one contiguous
# run.  Same bytes as the GGUF rows, permuted; a tile's record has the 16 rows' block size.
_Q6_SC = np.array([[0, 1, 4, 5], [2, 3, 6, 7], [8, 9, 12, 13], [10, 11, 14, 15]])   # lane kq's scale bytes


def pack_iq3s_tiled(raw_rows, kdim):
    """GGUF IQ3_S rows u8[N, 110*NB] (N % 16 == 0) -> tiled records u8[N/16, NB, 1760].

    Record (tile t, block b), row r = 16t + col, lane l = 16 kq + col: ``[0, 1024)`` lane l's 16 index
    bytes ``qs[16kq .. 16kq + 15]`` (block bytes 2..65); ``[1024, 1536)`` its 8 sign bytes
    ``signs[8kq ..]`` (bytes 74..105); ``[1536, 1664)`` its 2 high-bit bytes ``qh[2kq, 2kq + 1]``
    (bytes 66..73); ``[1664, 1728)`` its scale byte ``scales[kq]`` (bytes 106..109); ``[1728, 1760)``
    row col's d (bytes 0..1)."""
    x = np.ascontiguousarray(raw_rows, dtype=np.uint8)
    n, nb = len(x), kdim // 256
    assert n % 16 == 0 and x.shape[1] == 110 * nb
    blk = x.reshape(n // 16, 16, nb, 110).transpose(0, 2, 1, 3)             # [t, b, col, 110]
    def lanes(lo, per):                                                      # [t, b, kq, col, per]
        return blk[..., lo:lo + 4 * per].reshape(n // 16, nb, 16, 4, per).transpose(0, 1, 3, 2, 4)
    parts = [lanes(2, 16), lanes(74, 8), lanes(66, 2), lanes(106, 1)]
    flat = [a.reshape(n // 16, nb, -1) for a in parts] + [blk[..., 0:2].reshape(n // 16, nb, 32)]
    return np.ascontiguousarray(np.concatenate(flat, axis=2))


def unpack_iq3s_tiled(rec, kdim):
    """Inverse of :func:`pack_iq3s_tiled` -> GGUF IQ3_S rows u8[16*T, 110*NB]."""
    nb = kdim // 256
    r = np.ascontiguousarray(rec, dtype=np.uint8).reshape(-1, nb, 1760)
    t = len(r)
    def rows(lo, per):                                                       # -> [t, b, col, 4 per]
        return r[:, :, lo:lo + 64 * per].reshape(t, nb, 4, 16, per).transpose(0, 1, 3, 2, 4).reshape(t, nb, 16, 4 * per)
    blk = np.concatenate([r[:, :, 1728:1760].reshape(t, nb, 16, 2), rows(0, 16), rows(1536, 2), rows(1024, 8),
                          rows(1664, 1)], axis=3)                            # d, qs, qh, signs, scales
    return np.ascontiguousarray(blk.transpose(0, 2, 1, 3).reshape(16 * t, 110 * nb))


def pack_q6k_tiled(raw_rows, kdim):
    """GGUF Q6_K rows u8[N, 210*NB] (N % 16 == 0) -> tiled records u8[N/16, NB, 3360].

    Record (tile t, block b), row r = 16t + col, lane l = 16 kq + col: ``[0, 2048)`` lane l's 32 low
    bytes ``ql[32kq .. 32kq + 31]``; ``[2048, 3072)`` at ``32 (16h + col)`` row col's high bytes
    ``qh[32h .. 32h + 31]`` (h = 0, 1); ``[3072, 3328)`` lane l's 4 scale bytes ``sc[8h + 2c + {0, 1,
    4, 5}]`` (h = kq / 2, c = kq % 2); ``[3328, 3360)`` row col's d (bytes 208..209)."""
    x = np.ascontiguousarray(raw_rows, dtype=np.uint8)
    n, nb = len(x), kdim // 256
    assert n % 16 == 0 and x.shape[1] == 210 * nb
    blk = x.reshape(n // 16, 16, nb, 210).transpose(0, 2, 1, 3)             # [t, b, col, 210]
    ql = blk[..., 0:128].reshape(n // 16, nb, 16, 4, 32).transpose(0, 1, 3, 2, 4)
    qh = blk[..., 128:192].reshape(n // 16, nb, 16, 2, 32).transpose(0, 1, 3, 2, 4)
    sc = blk[..., 192 + _Q6_SC].transpose(0, 1, 3, 2, 4)                     # [t, b, kq, col, 4]
    flat = [a.reshape(n // 16, nb, -1) for a in (ql, qh, sc)] + [blk[..., 208:210].reshape(n // 16, nb, 32)]
    return np.ascontiguousarray(np.concatenate(flat, axis=2))


def unpack_q6k_tiled(rec, kdim):
    """Inverse of :func:`pack_q6k_tiled` -> GGUF Q6_K rows u8[16*T, 210*NB]."""
    nb = kdim // 256
    r = np.ascontiguousarray(rec, dtype=np.uint8).reshape(-1, nb, 3360)
    t = len(r)
    ql = r[:, :, 0:2048].reshape(t, nb, 4, 16, 32).transpose(0, 1, 3, 2, 4).reshape(t, nb, 16, 128)
    qh = r[:, :, 2048:3072].reshape(t, nb, 2, 16, 32).transpose(0, 1, 3, 2, 4).reshape(t, nb, 16, 64)
    scl = r[:, :, 3072:3328].reshape(t, nb, 4, 16, 4).transpose(0, 1, 3, 2, 4)   # [t, b, col, kq, 4]
    sc = np.empty((t, nb, 16, 16), dtype=np.uint8)
    sc[..., _Q6_SC] = scl
    d = r[:, :, 3328:3360].reshape(t, nb, 16, 2)
    blk = np.concatenate([ql, qh, sc, d], axis=3)
    return np.ascontiguousarray(blk.transpose(0, 2, 1, 3).reshape(16 * t, 210 * nb))
