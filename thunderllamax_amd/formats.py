"""Host-side weight formats: the reference's repacked layouts and its table buffers.

The kernels consume the layouts the reference's engine uploads:

* IQ3_XXS "packed" rows (/root/reference/engine/pack_w1c.py:18-31): per row
  ``[qs 64*NB][sw 32*NB][d 2*NB]`` -- the same 98*NB bytes as the GGUF row, regrouped so
  each field is naturally aligned;
* Q6_K padded 212-B blocks (/root/reference/engine/pack_w1c.py:33-45)
  ``[pad 2][d 2][sc 16][ql 128][qh 64]``;
* IQ3_XXS packed7 16-B units (/root/reference/engine/pack_w7.py:7-15).

All three are pure byte permutations of the GGUF data, computed here with array reshapes.
"""
import numpy as np

from .tables import iq3xxs_gridf, iq3xxs_lut8, iq4nl_f32

IQ3XXS_BLOCK = 98
Q6K_BLOCK = 210
Q6K_PAD_BLOCK = 212
IQ4XS_BLOCK = 136


def iq3_pack_rows(raw, kdim):
    """GGUF IQ3_XXS rows u8[N, 98*NB] -> packed rows (same size)."""
    nb = kdim // 256
    blk = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, nb, IQ3XXS_BLOCK)
    # field-major concatenation: all qs, then all scale words, then all d
    return np.concatenate([blk[:, :, 2:66].reshape(len(blk), -1),
                           blk[:, :, 66:98].reshape(len(blk), -1),
                           blk[:, :, 0:2].reshape(len(blk), -1)], axis=1)


def q6_pad_rows(raw, kdim):
    """GGUF Q6_K rows u8[N, 210*NB] -> padded rows u8[N, 212*NB]."""
    nb = kdim // 256
    blk = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, nb, Q6K_BLOCK)
    n = len(blk)
    pad = np.zeros((n, nb, 2), dtype=np.uint8)
    out = np.concatenate([pad, blk[:, :, 208:210], blk[:, :, 192:208], blk[:, :, 0:192]], axis=2)
    return out.reshape(n, nb * Q6K_PAD_BLOCK)


def iq3_pack7(packed, kdim):
    """Packed IQ3_XXS rows u8[N, 98*NB] (N % 8 == 0) -> packed7 units u8[N/8, K/128, 32, 16]."""
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    n = len(p)
    nb = kdim // 256
    q = p[:, :64 * nb].view("<u2").reshape(n, nb, 2, 4, 4)        # [row, b, h, c, cc]
    sw = p[:, 64 * nb:96 * nb].view("<u4").reshape(n, nb, 2, 4)   # [row, b, h, c]
    d = p[:, 96 * nb:98 * nb].view("<u2").reshape(n, nb)          # [row, b]
    unit = np.zeros((n, nb, 2, 4, 8), dtype="<u2")
    unit[..., 0:4] = q
    unit[..., 4] = (sw & 0xFFFF).astype("<u2")
    unit[..., 5] = (sw >> 16).astype("<u2")
    unit[..., 6] = d[:, :, None, None]
    # [group, r, b, h, c, 8] -> [group, chunk=(b,h), r, c, 8]
    unit = unit.reshape(n // 8, 8, nb, 2, 4, 8).transpose(0, 2, 3, 1, 4, 5)
    return np.ascontiguousarray(unit).view(np.uint8).reshape(n // 8, nb * 2, 32, 16)


def gridf_tensor(device="cuda"):
    """The ``gridf`` buffer (float32[1024]) every IQ3_XXS entry point takes."""
    import torch
    return torch.from_numpy(iq3xxs_gridf()).to(device)


def lut8_tensor(device="cuda"):
    """The ``lut8`` buffer (int8[1024]) of the W4A8 prefill branch."""
    import torch
    return torch.from_numpy(iq3xxs_lut8()).to(device)


def iq4nl_tensor(device="cuda"):
    """The IQ4_NL level buffer (float32[16])."""
    import torch
    return torch.from_numpy(iq4nl_f32()).to(device)


def pointer_table(tensors, device="cuda"):
    """Device int64 array of the tensors' device addresses (the MoE per-expert slab table)."""
    import torch
    return torch.tensor([t.data_ptr() for t in tensors], dtype=torch.int64, device=device)
