"""Python mirror of the reference's kernel call sites, running on libtlx_hip.

Each function keeps the reference kernel's name and positional argument order
(``ffn8(wg, wu, gridf, hhx, gact)`` etc., /root/reference/engine/ffn8.cu:134-136) and takes
torch tensors on the GPU.  Sizes the reference bakes into kernel names (M, N, K) are read
from the tensor shapes.  Like the reference, the output buffers are caller-owned; nothing is
allocated here.  Errors raise ``TlxError`` (the reference asserts in Python).
"""
import torch

from ._lib import LAYOUT_PACK7, LAYOUT_PACKED, LAYOUT_RAW, call

_F16 = torch.float16


def _stream(stream):
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return getattr(stream, "cuda_stream", stream)


def _dev(*ts):
    for t in ts:
        if not (t.is_cuda and t.is_contiguous()):
            raise ValueError("all buffers must be contiguous tensors on the GPU")


def _mk(x):
    """[K] or [M, K] activations -> M."""
    return 1 if x.dim() == 1 else x.shape[0]


# ------------------------------------------------------------------ dequantization
def iq3xxs_dequant(w, gridf, out, kdim, layout=LAYOUT_PACKED, stream=None):
    _dev(w, gridf, out)
    rows = w.numel() // (98 * (kdim // 256))
    call("tlx_iq3xxs_dequant", w.data_ptr(), gridf.data_ptr(), out.data_ptr(), rows, kdim, layout,
         int(out.dtype == _F16), _stream(stream))
    return out


def q6k_dequant(w, out, kdim, layout=LAYOUT_RAW, stream=None):
    _dev(w, out)
    bs = 210 if layout == LAYOUT_RAW else 212
    rows = w.numel() // (bs * (kdim // 256))
    call("tlx_q6k_dequant", w.data_ptr(), out.data_ptr(), rows, kdim, layout, int(out.dtype == _F16),
         _stream(stream))
    return out


def iq4xs_dequant(w, iq4nl, out, kdim, stream=None):
    _dev(w, iq4nl, out)
    rows = w.numel() // (136 * (kdim // 256))
    call("tlx_iq4xs_dequant", w.data_ptr(), iq4nl.data_ptr(), out.data_ptr(), rows, kdim, _stream(stream))
    return out


# ------------------------------------------------------------------ decode GEMVs
def ffn8(wg, wu, gridf, hhx, gact, layout=LAYOUT_PACKED, stream=None):
    """gact[m] = silu16(half(Wg·hhx[m])) * half(Wu·hhx[m])   (ffn8 / ffn8v{M})."""
    _dev(wg, wu, gridf, hhx, gact)
    M, K, N = _mk(hhx), hhx.shape[-1], gact.shape[-1]
    call("tlx_ffn8", wg.data_ptr(), wu.data_ptr(), gridf.data_ptr(), hhx.data_ptr(), gact.data_ptr(),
         M, N, K, layout, _stream(stream))
    return gact


def down8(wd, gridf, gact, hh, y, layout=LAYOUT_PACKED, stream=None):
    """y[m] = hh[m] + float(half(Wd·gact[m]))   (down8 / down8nw32_{M})."""
    _dev(wd, gridf, gact, hh, y)
    M, K, N = _mk(gact), gact.shape[-1], y.shape[-1]
    call("tlx_down8", wd.data_ptr(), gridf.data_ptr(), gact.data_ptr(), hh.data_ptr(), y.data_ptr(),
         M, N, K, layout, _stream(stream))
    return y


def iq3_gemv(w, gridf, x, out, layout=LAYOUT_PACKED, stream=None):
    """out[m] = half(W·x[m])   (the IQ3ROWP segment body)."""
    _dev(w, gridf, x, out)
    M, K, N = _mk(x), x.shape[-1], out.shape[-1]
    call("tlx_iq3_gemv", w.data_ptr(), gridf.data_ptr(), x.data_ptr(), out.data_ptr(), M, N, K, layout,
         _stream(stream))
    return out


def aq3k8(wq, wk, wv, gridf, xh, qrow, krow, vrow, layout=LAYOUT_PACKED, stream=None):
    """Fused q/k/v IQ3_XXS projections in one launch   (aq3k8 / aq3k8v{M})."""
    _dev(wq, wk, wv, gridf, xh, qrow, krow, vrow)
    M, K = _mk(xh), xh.shape[-1]
    call("tlx_aq3k8", wq.data_ptr(), wk.data_ptr(), wv.data_ptr(), gridf.data_ptr(), xh.data_ptr(),
         qrow.data_ptr(), krow.data_ptr(), vrow.data_ptr(), M, qrow.shape[-1], krow.shape[-1],
         vrow.shape[-1], K, layout, _stream(stream))


def h6k_gemv(w, x, y, layout=LAYOUT_RAW, stream=None):
    """y = W·x, Q6_K weights, fp32 x and y   (h6k2048 contract)."""
    _dev(w, x, y)
    call("tlx_q6k_gemv", w.data_ptr(), x.data_ptr(), y.data_ptr(), y.numel(), x.numel(), layout,
         _stream(stream))
    return y


# ------------------------------------------------------------------ prefill dequant-GEMMs
# Weights are IQ3_XXS in the packed7 unit layout (``formats.iq3_pack7``), as the reference's
# prefill GEMMs read them.
def pfg3_ffn(wg, wu, gridf, x16, out16, layout=LAYOUT_PACK7, stream=None):
    """out16[m] = silu16(half(Wg·x16[m])) * half(Wu·x16[m]) over a prompt chunk
    (pf_gemm3 FFN=1: kernel(w1, w2, gridf, x16, out16))."""
    _dev(wg, wu, gridf, x16, out16)
    M, K, N = x16.shape[0], x16.shape[1], out16.shape[1]
    call("tlx_pfg3_ffn", wg.data_ptr(), wu.data_ptr(), gridf.data_ptr(), x16.data_ptr(), out16.data_ptr(),
         M, N, K, layout, _stream(stream))
    return out16


def pfg3_iq3d(w, gridf, x16, res16, out32, layout=LAYOUT_PACK7, stream=None):
    """out32[m] = res16[m] + W·x16[m]   (pf_gemm3 RES=1: kernel(w1, gridf, x16, res16, out32))."""
    _dev(w, gridf, x16, res16, out32)
    M, K, N = x16.shape[0], x16.shape[1], out32.shape[1]
    call("tlx_pfg3_iq3d", w.data_ptr(), gridf.data_ptr(), x16.data_ptr(), res16.data_ptr(), out32.data_ptr(),
         M, N, K, layout, _stream(stream))
    return out32


def pfg3_iq3o(w, gridf, x16, out16, layout=LAYOUT_PACK7, stream=None):
    """out16[m] = half(W·x16[m])   (pf_gemm3 plain: kernel(w1, gridf, x16, out16))."""
    _dev(w, gridf, x16, out16)
    M, K, N = x16.shape[0], x16.shape[1], out16.shape[1]
    call("tlx_pfg3_iq3o", w.data_ptr(), gridf.data_ptr(), x16.data_ptr(), out16.data_ptr(), M, N, K, layout,
         _stream(stream))
    return out16


# ------------------------------------------------------------------ MoE grouped experts
# 256 routed experts + 1 shared, hidden 2048, expert intermediate 512, top-8, IQ4_XS weights.
# ptbl / ptbl_dn: int64 device tensors of 256 slab addresses (formats.pointer_table).
def moe_topk(logits, eids, gates, stream=None):
    """Top-8 + renormalized softmax from router logits [P][256] (the rt8e256 epilogue)."""
    _dev(logits, eids, gates)
    call("tlx_moe_topk", logits.data_ptr(), eids.data_ptr(), gates.data_ptr(), logits.shape[0], _stream(stream))


def moe_route(wrt, wsh, h, eids, gates, sg, stream=None):
    """rt8e256(wrt, wsh, h, eids, gates, sg)."""
    _dev(wrt, wsh, h, eids, gates, sg)
    call("tlx_moe_route", wrt.data_ptr(), wsh.data_ptr(), h.data_ptr(), eids.data_ptr(), gates.data_ptr(),
         sg.data_ptr(), h.shape[0], _stream(stream))


def moe_max_items(npair):
    from ._lib import lib
    return lib().tlx_moe_max_items(npair)


def moe_sort(eids, eoff, plist, items, nitp, stream=None):
    """mmsort8(eids, eoff, plist, items, nitp, np) with np = eids.numel()."""
    _dev(eids, eoff, plist, items, nitp)
    call("tlx_moe_sort", eids.data_ptr(), eoff.data_ptr(), plist.data_ptr(), items.data_ptr(), nitp.data_ptr(),
         eids.numel(), _stream(stream))


def moe_up4(ptbl, eoff, plist, items, nitp, xs, iq4nl, ys, stream=None):
    """ys[pair][512] = silu(Wg_e . x[pos]) * (Wu_e . x[pos])   (gx8e256up4 / gxu_gm)."""
    _dev(ptbl, eoff, plist, items, nitp, xs, iq4nl, ys)
    call("tlx_moe_up4", ptbl.data_ptr(), eoff.data_ptr(), plist.data_ptr(), items.data_ptr(), nitp.data_ptr(),
         xs.data_ptr(), iq4nl.data_ptr(), ys.data_ptr(), ys.shape[0], _stream(stream))


def moe_dn4(ptbl_dn, eoff, plist, items, nitp, act, iq4nl, parts, stream=None):
    """parts[pair][2048] = fp16(Wd_e . act[pair])   (gx8e256dn / gxd_gm)."""
    _dev(ptbl_dn, eoff, plist, items, nitp, act, iq4nl, parts)
    call("tlx_moe_dn4", ptbl_dn.data_ptr(), eoff.data_ptr(), plist.data_ptr(), items.data_ptr(), nitp.data_ptr(),
         act.data_ptr(), iq4nl.data_ptr(), parts.data_ptr(), act.shape[0], _stream(stream))


def moe_shared(ptbl_sh, xs, iq4nl, act, out, stream=None):
    """Shared expert over all positions: act [P][512] (scratch), out [P][2048] f32."""
    _dev(ptbl_sh, xs, iq4nl, act, out)
    call("tlx_moe_shared", ptbl_sh.data_ptr(), xs.data_ptr(), iq4nl.data_ptr(), act.data_ptr(), out.data_ptr(),
         xs.shape[0], _stream(stream))


def moe_combine(parts, gates, sg, shared, hres, y, stream=None):
    """cmbz2048(parts, gates, sg, shared, hres, y)."""
    _dev(parts, gates, sg, shared, hres, y)
    call("tlx_moe_combine", parts.data_ptr(), gates.data_ptr(), sg.data_ptr(), shared.data_ptr(), hres.data_ptr(),
         y.data_ptr(), y.shape[0], _stream(stream))
