"""numpy restatements of the reference's weight repackers (pure byte permutations).

* ``pack_iq3_w1c``  -- /root/reference/engine/pack_w1c.py:18-31  raw IQ3_XXS rows -> packed rows
* ``pack_q6_pad``   -- /root/reference/engine/pack_w1c.py:33-45  raw Q6_K rows -> 212-B blocks
* ``pack_w7``       -- /root/reference/engine/pack_w7.py:40-73   packed IQ3 rows -> packed7 units
* ``unpack_w7``     -- /root/reference/engine/pack_w7.py:75-96   the inverse
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
