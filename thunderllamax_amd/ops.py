"""Python mirror of the reference's kernel call sites, running on libtlx_hip.

Each function keeps the reference kernel's name and positional argument order
(``ffn8(wg, wu, gridf, hhx, gact)`` etc., /root/reference/engine/ffn8.cu:134-136) and takes
torch tensors on the GPU.  Sizes the reference bakes into kernel names (M, N, K) are read
from the tensor shapes.  Like the reference, the output buffers are caller-owned; nothing is
allocated here.  Errors raise ``TlxError`` (the reference asserts in Python).
"""
import torch

from ._lib import IN_TILEORD, LAYOUT_PACK7, LAYOUT_PACKED, LAYOUT_RAW, LAYOUT_TILED, OUT_TILEORD, V_Q4K, call

_F16 = torch.float16

# ------------------------------------------------------------------ workspaces
# The library allocates no device memory: its scratch buffers are caller-owned and attached per
# device (tlx_attach_workspace), as the reference's host allocates every buffer once at boot
# (/root/reference/engine/engine0.py:85-95).  This module owns one pair per device.
_WORKSPACES = {}


def workspace_sizes():
    """(GEMV workspace bytes, prefill-GEMM split workspace bytes) the library asks for."""
    import ctypes
    g, m = ctypes.c_uint64(), ctypes.c_uint64()
    call("tlx_workspace_size", ctypes.byref(g), ctypes.byref(m))
    return g.value, m.value


def attach_workspace(device=None, gemm_bytes=None, stream=None):
    """Allocate the library's scratch buffers on `device` (default: the current device) with torch
    and attach them: the GEMV workspace (zeroed counters) and the prefill GEMM's split workspace
    (``gemm_bytes``, default the library's full size; 0 = none, the GEMMs then run whole tiles).
    Call it outside stream capture; the ops below attach on the first use of a device."""
    dev = torch.device("cuda", torch.cuda.current_device() if device is None else torch.device(device).index)
    gb, mb = workspace_sizes()
    mb = mb if gemm_bytes is None else int(gemm_bytes)
    with torch.cuda.device(dev):
        g = torch.zeros(gb, dtype=torch.uint8, device=dev)
        m = torch.empty(mb, dtype=torch.uint8, device=dev) if mb > 0 else None
        call("tlx_attach_workspace", g.data_ptr(), gb, None if m is None else m.data_ptr(), mb,
             _stream(stream))
        # the fill (torch's current stream) and the counter clear (`stream`) complete before any
        # call on any stream can use the workspace: a call on another stream that overlapped the
        # clear could leave an arrival counter at 1 for every later call on the device
        torch.cuda.synchronize(dev)
    _WORKSPACES[dev.index] = (g, m)
    return g, m


def _ws(t):
    """Attach the workspaces of t's device on its first use there (never inside stream capture:
    an allocation there would belong to the graph).  Every wrapper calls it before its first
    launch, so the library's one-time set-up (kernel attributes) also runs outside capture."""
    if t.device.index in _WORKSPACES:
        return
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("libtlx workspace not attached on this device: call ops.attach_workspace() "
                           "before capturing a graph")
    attach_workspace(t.device)


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


def tileord_empty(n, device, dtype=torch.float16):
    """A buffer for n activations in the tile-ordered form [n/8][16][8] (the form in which the
    IQ3_XXS GEMVs read activations without a copy launch; slot r holds row r, rows M..15 repeat
    row M-1), for TLX_OUT_TILEORD outputs / TLX_IN_TILEORD inputs."""
    if n % 8:
        raise ValueError("the tile-ordered form needs a multiple of 8 columns")
    return torch.empty(n // 8, 16, 8, dtype=dtype, device=device)


def tileord_to_rows(t, m):
    """The first m rows of a tile-ordered [n/8][16][8] buffer as a row-major [m][n] tensor."""
    return t.permute(1, 0, 2).reshape(16, -1)[:m]


def _tileord_n(t):
    """Columns of a tile-ordered [n/8][16][8] buffer."""
    if t.dim() != 3 or t.shape[1:] != (16, 8):
        raise ValueError("a tile-ordered buffer is [n/8][16][8]")
    return t.shape[0] * 8


def _need(t, nbytes, what):
    """Raise unless buffer `t` holds at least `nbytes` bytes: the library sees only pointers,
    so a buffer too small for the shape and layout it is described with must be caught here."""
    have = t.numel() * t.element_size()
    if have < nbytes:
        raise ValueError(f"{what}: {have} bytes, the call needs {nbytes}")


def _iq3_rows(n, k):
    return n * 98 * (k // 256)


def _iq3_w(n, k, layout):
    """Bytes of an IQ3_XXS matrix of n rows in `layout` (tiled: 102-B records of whole 16-row
    tiles; packed7: 16-B units, 128 B per 256 weights)."""
    if layout == LAYOUT_TILED:
        return (n + 15) // 16 * 16 * 102 * (k // 256)
    if layout == LAYOUT_PACK7:
        return _pack7(n, k)
    return _iq3_rows(n, k)


def _pack7(n, k):
    return n * (k // 2)


# ------------------------------------------------------------------ dequantization
def iq3xxs_dequant(w, gridf, out, kdim, layout=LAYOUT_PACKED, stream=None):
    rows = w.numel() * w.element_size() // (98 * (kdim // 256))
    _need(out, rows * kdim * out.element_size(), "out")
    _need(gridf, 4096, "gridf")
    _dev(w, gridf, out)
    call("tlx_iq3xxs_dequant", w.data_ptr(), gridf.data_ptr(), out.data_ptr(), rows, kdim, layout,
         int(out.dtype == _F16), _stream(stream))
    return out


def q6k_dequant(w, out, kdim, layout=LAYOUT_RAW, stream=None):
    bs = 210 if layout == LAYOUT_RAW else 212
    rows = w.numel() * w.element_size() // (bs * (kdim // 256))
    _need(out, rows * kdim * out.element_size(), "out")
    _dev(w, out)
    call("tlx_q6k_dequant", w.data_ptr(), out.data_ptr(), rows, kdim, layout, int(out.dtype == _F16),
         _stream(stream))
    return out


def iq4xs_dequant(w, iq4nl, out, kdim, stream=None):
    rows = w.numel() * w.element_size() // (136 * (kdim // 256))
    _need(out, rows * kdim * 4, "out")
    _need(iq4nl, 64, "iq4nl")
    _dev(w, iq4nl, out)
    call("tlx_iq4xs_dequant", w.data_ptr(), iq4nl.data_ptr(), out.data_ptr(), rows, kdim, _stream(stream))
    return out


def iq3s_dequant(w, gridf, out, kdim, stream=None):
    """IQ3_S rows (110 B per 256 weights) -> f32 or f16 ``out`` (bit-exact GGUF values); gridf:
    the 512-entry grid as float[512][4] (a run-time table, as the reference passes it)."""
    rows = w.numel() * w.element_size() // (110 * (kdim // 256))
    _need(out, rows * kdim * out.element_size(), "out")
    _need(gridf, 512 * 16, "gridf")
    _dev(w, gridf, out)
    call("tlx_iq3s_dequant", w.data_ptr(), gridf.data_ptr(), out.data_ptr(), rows, kdim, int(out.dtype == _F16),
         _stream(stream))
    return out


def q8_0_dequant(w, out, kdim, stream=None):
    """Q8_0 rows (34 B per 32 weights) -> f32 or f16 ``out`` (bit-exact d * q)."""
    rows = w.numel() * w.element_size() // (34 * (kdim // 32))
    _need(out, rows * kdim * out.element_size(), "out")
    _dev(w, out)
    call("tlx_q8_0_dequant", w.data_ptr(), out.data_ptr(), rows, kdim, int(out.dtype == _F16), _stream(stream))
    return out


# ------------------------------------------------------------------ decode GEMVs
def ffn8(wg, wu, gridf, hhx, gact, layout=LAYOUT_PACKED, stream=None, out_tileord=False, in_tileord=False,
         m=None):
    """gact[m] = silu16(half(Wg·hhx[m])) * half(Wu·hhx[m])   (ffn8 / ffn8v{M}).  With
    ``out_tileord`` (tiled records only) gact is a tile-ordered [N/8][16][8] buffer (tileord_empty),
    which down8 / iq3_gemv read with ``in_tileord`` and no copy launch; with ``in_tileord`` hhx is
    such a buffer (then M is given by ``m`` or gact's rows)."""
    K = _tileord_n(hhx) if in_tileord else hhx.shape[-1]
    N = _tileord_n(gact) if out_tileord else gact.shape[-1]
    M = m if m is not None else (_mk(hhx) if not in_tileord else _mk(gact) if not out_tileord else None)
    if M is None:
        raise ValueError("both sides tile-ordered: pass m")
    _need(wg, _iq3_w(N, K, layout), "wg")
    _need(wu, _iq3_w(N, K, layout), "wu")
    _need(gridf, 4096, "gridf")
    _need(hhx, (16 if in_tileord else M) * K * 2, "hhx")
    _need(gact, (16 if out_tileord else M) * N * 2, "gact")
    _dev(wg, wu, gridf, hhx, gact)
    _ws(wg)
    fl = (IN_TILEORD if in_tileord else 0) | (OUT_TILEORD if out_tileord else 0)
    call("tlx_ffn8", wg.data_ptr(), wu.data_ptr(), gridf.data_ptr(), hhx.data_ptr(), gact.data_ptr(),
         M, N, K, layout | fl, _stream(stream))
    return gact


def ffn8_noalloc(wg, wu, gridf, hhx, gact, layout=LAYOUT_PACKED, stream=None):
    """ffn8 on the library's own fixed scratch: no workspace, no allocation (for callers that
    cannot allocate; calls overlapping in time on one device race on that scratch)."""
    M, K, N = _mk(hhx), hhx.shape[-1], gact.shape[-1]
    _need(wg, _iq3_w(N, K, layout), "wg")
    _need(wu, _iq3_w(N, K, layout), "wu")
    _need(gridf, 4096, "gridf")
    _need(gact, M * N * 2, "gact")
    _dev(wg, wu, gridf, hhx, gact)
    call("tlx_ffn8_noalloc", wg.data_ptr(), wu.data_ptr(), gridf.data_ptr(), hhx.data_ptr(), gact.data_ptr(),
         M, N, K, layout, _stream(stream))
    return gact


def rms_f16(x, nw, xh, stream=None):
    """xh[m] = half((x[m] * r) * nw), r = rsqrt(mean(x[m]^2) + 1e-6)   (k0n{M} / k0_norm)."""
    M, D = x.shape
    _need(nw, D * 4, "nw")
    _need(xh, M * D * 2, "xh")
    _dev(x, nw, xh)
    call("tlx_rms_f16", x.data_ptr(), nw.data_ptr(), xh.data_ptr(), M, D, _stream(stream))
    return xh


def add_rms_f16(x, a, nw, hh, hhx, stream=None):
    """hh = x + float(a); hhx[m] = half((hh[m] * r) * nw)   (hh{M} / k3m_hh)."""
    M, D = x.shape
    _need(a, M * D * 2, "a")
    _need(nw, D * 4, "nw")
    _need(hh, M * D * 4, "hh")
    _need(hhx, M * D * 2, "hhx")
    _dev(x, a, nw, hh, hhx)
    call("tlx_add_rms_f16", x.data_ptr(), a.data_ptr(), nw.data_ptr(), hh.data_ptr(), hhx.data_ptr(), M, D,
         _stream(stream))
    return hh, hhx


def ffn8_hh(wg, wu, gridf, x, attn_out, nw2, hh, hhx, gact, layout=LAYOUT_PACKED, stream=None):
    """hh{M} + ffn8 in one call: hh = x + float(attn_out), hhx = norm(hh), gact = ffn8(hhx)."""
    M, K, N = x.shape[0], x.shape[1], gact.shape[-1]
    _need(wg, _iq3_w(N, K, layout), "wg")
    _need(wu, _iq3_w(N, K, layout), "wu")
    _need(gridf, 4096, "gridf")
    _need(attn_out, M * K * 2, "attn_out")
    _need(nw2, K * 4, "nw2")
    _need(hh, M * K * 4, "hh")
    _need(hhx, M * K * 2, "hhx")
    _need(gact, M * N * 2, "gact")
    _dev(wg, wu, gridf, x, attn_out, nw2, hh, hhx, gact)
    _ws(wg)
    call("tlx_ffn8_hh", wg.data_ptr(), wu.data_ptr(), gridf.data_ptr(), x.data_ptr(), attn_out.data_ptr(),
         nw2.data_ptr(), hh.data_ptr(), hhx.data_ptr(), gact.data_ptr(), M, N, K, layout, _stream(stream))
    return gact


def down8(wd, gridf, gact, hh, y, layout=LAYOUT_PACKED, stream=None, in_tileord=False):
    """y[m] = hh[m] + float(half(Wd·gact[m]))   (down8 / down8nw32_{M}).  With ``in_tileord``
    gact is a tile-ordered [K/8][16][8] buffer (e.g. ffn8's ``out_tileord`` output) and M = y's rows."""
    if in_tileord:
        M, K = _mk(y), _tileord_n(gact)
    else:
        M, K = _mk(gact), gact.shape[-1]
    N = y.shape[-1]
    _need(wd, _iq3_w(N, K, layout), "wd")
    _need(gridf, 4096, "gridf")
    _need(gact, (16 if in_tileord else M) * K * 2, "gact")
    _need(hh, M * N * 4, "hh")
    _need(y, M * N * 4, "y")
    _dev(wd, gridf, gact, hh, y)
    _ws(wd)
    call("tlx_down8", wd.data_ptr(), gridf.data_ptr(), gact.data_ptr(), hh.data_ptr(), y.data_ptr(),
         M, N, K, layout | (IN_TILEORD if in_tileord else 0), _stream(stream))
    return y


def iq3_gemv(w, gridf, x, out, layout=LAYOUT_PACKED, stream=None, in_tileord=False, out_tileord=False, m=None):
    """out[m] = half(W·x[m])   (the IQ3ROWP segment body).  ``in_tileord`` / ``out_tileord``: x / out
    in the tile-ordered [n/8][16][8] form (then M is given by ``m`` or the row-major side)."""
    K = _tileord_n(x) if in_tileord else x.shape[-1]
    N = _tileord_n(out) if out_tileord else out.shape[-1]
    M = m if m is not None else (_mk(x) if not in_tileord else _mk(out) if not out_tileord else None)
    if M is None:
        raise ValueError("both sides tile-ordered: pass m")
    _need(w, _iq3_w(N, K, layout), "w")
    _need(gridf, 4096, "gridf")
    _need(x, (16 if in_tileord else M) * K * 2, "x")
    _need(out, (16 if out_tileord else M) * N * 2, "out")
    _dev(w, gridf, x, out)
    _ws(w)
    fl = (IN_TILEORD if in_tileord else 0) | (OUT_TILEORD if out_tileord else 0)
    call("tlx_iq3_gemv", w.data_ptr(), gridf.data_ptr(), x.data_ptr(), out.data_ptr(), M, N, K, layout | fl,
         _stream(stream))
    return out


def iq3_gemv_multi(ws, gridf, x, outs, layout=LAYOUT_PACKED, stream=None):
    """outs[s][m] = half(W_s·x[m]) for up to four IQ3_XXS matrices sharing x, one launch (the GDN
    block's qkv / gate / alpha / beta projections, engine/gdn_block.cu:44-148)."""
    import ctypes
    if not 1 <= len(ws) == len(outs) <= 4:
        raise ValueError("one to four matrices, one output each")
    M, K = _mk(x), x.shape[-1]
    for i, (w, o) in enumerate(zip(ws, outs)):
        _need(w, _iq3_w(o.shape[-1], K, layout), f"w[{i}]")
        _need(o, M * o.shape[-1] * 2, f"out[{i}]")
    _need(gridf, 4096, "gridf")
    _dev(*ws, *outs, gridf, x)
    k = len(ws)
    wp = (ctypes.c_void_p * k)(*[w.data_ptr() for w in ws])
    op = (ctypes.c_void_p * k)(*[o.data_ptr() for o in outs])
    n = (ctypes.c_int * k)(*[o.shape[-1] for o in outs])
    _ws(x)
    call("tlx_iq3_gemv_multi", wp, op, n, k, gridf.data_ptr(), x.data_ptr(), M, K, layout, _stream(stream))
    return outs


def _q4k_rows(n, k):
    return n * 144 * (k // 256)


def _attn(name, wq, wk, wv, gridf, xh, qrow, krow, vrow, qbytes, kbytes, vbytes, layout, stream):
    M, K = _mk(xh), xh.shape[-1]
    for t, o, nm, nbytes in ((wq, qrow, "wq", qbytes), (wk, krow, "wk", kbytes), (wv, vrow, "wv", vbytes)):
        _need(t, nbytes(o.shape[-1], K), nm)
        _need(o, M * o.shape[-1] * 2, nm + " output")
    _need(gridf, 4096, "gridf")
    _dev(wq, wk, wv, gridf, xh, qrow, krow, vrow)
    args = [wq.data_ptr(), wk.data_ptr(), wv.data_ptr(), gridf.data_ptr(), xh.data_ptr(),
            qrow.data_ptr(), krow.data_ptr(), vrow.data_ptr(), M, qrow.shape[-1], krow.shape[-1],
            vrow.shape[-1], K]
    if layout is not None:
        args.append(layout)
    _ws(xh)
    call(name, *args, _stream(stream))


def aq3k8(wq, wk, wv, gridf, xh, qrow, krow, vrow, layout=LAYOUT_PACKED, stream=None):
    """Fused q/k/v projections (aq3k8 / aq3k8v{M}): q, k IQ3_XXS in ``layout`` (packed rows, GGUF
    blocks or tiled records); v IQ3_XXS too, or GGUF Q4_K when ``layout`` includes ``V_Q4K``."""
    base = layout & ~V_Q4K
    iq3 = lambda n, k: _iq3_w(n, k, base)   # noqa: E731
    v = _q4k_rows if layout & V_Q4K else iq3
    _attn("tlx_aq3k8", wq, wk, wv, gridf, xh, qrow, krow, vrow, iq3, iq3, v, layout, stream)


def a_qkv_iq3(wq, wk, wv4, gridf, xh, qrow, krow, vrow, stream=None):
    """Fused q/k/v projections on GGUF blocks (a_qkv_iq3): q, k IQ3_XXS, v Q4_K."""
    _attn("tlx_a_qkv_iq3", wq, wk, wv4, gridf, xh, qrow, krow, vrow, _iq3_rows, _iq3_rows, _q4k_rows,
          None, stream)


def a_qkv_q6(wq, wk, wv4, gridf, xh, qrow, krow, vrow, stream=None):
    """Fused q/k/v projections on GGUF blocks (a_qkv_q6): q Q6_K (210-B), k IQ3_XXS, v Q4_K."""
    _attn("tlx_a_qkv_q6", wq, wk, wv4, gridf, xh, qrow, krow, vrow,
          lambda n, k: _q6_rows(n, k, LAYOUT_RAW), _iq3_rows, _q4k_rows, None, stream)


def h6k_gemv(w, x, y, layout=LAYOUT_RAW, stream=None):
    """y = W·x, Q6_K weights, fp32 x and y   (h6k2048 contract)."""
    _need(w, y.numel() * (210 if layout == LAYOUT_RAW else 212) * (x.numel() // 256), "w")
    _dev(w, x, y)
    _ws(w)
    call("tlx_q6k_gemv", w.data_ptr(), x.data_ptr(), y.data_ptr(), y.numel(), x.numel(), layout,
         _stream(stream))
    return y


def _q6_rows(n, k, layout):
    return n * (210 if layout == LAYOUT_RAW else 212) * (k // 256)


def q6k_gemv16(w, x, out, layout=LAYOUT_PACKED, stream=None):
    """out[m][n] = half(W[n]·x[m]), Q6_K weights (raw 210-B or padded 212-B blocks), fp16
    activations and outputs (the q-branch body of aq6k8 / a_qkv_q6 and the Q6_K head)."""
    M, K = x.shape
    N = out.shape[-1]
    _need(w, _q6_rows(N, K, layout), "w")
    _need(out, M * N * 2, "out")
    _dev(w, x, out)
    _ws(w)
    call("tlx_q6k_gemv16", w.data_ptr(), x.data_ptr(), out.data_ptr(), M, N, K, layout,
         _stream(stream))
    return out


def _k4_gemv(name, nbytes, w, x, out, stream):
    M, K = x.shape
    N = out.shape[-1]
    _need(w, N * nbytes * (K // 256), "w")
    _need(out, M * N * 2, "out")
    _dev(w, x, out)
    _ws(w)
    call(name, w.data_ptr(), x.data_ptr(), out.data_ptr(), M, N, K, _stream(stream))
    return out


def q4k_gemv16(w, x, out, stream=None):
    """out[m][n] = half(W[n]·x[m]), GGUF Q4_K rows (144-B blocks), fp16 x and out."""
    return _k4_gemv("tlx_q4k_gemv16", 144, w, x, out, stream)


def q5k_gemv16(w, x, out, stream=None):
    """out[m][n] = half(W[n]·x[m]), GGUF Q5_K rows (176-B blocks), fp16 x and out."""
    return _k4_gemv("tlx_q5k_gemv16", 176, w, x, out, stream)


def head8(wq5, xh, logits, stream=None):
    """Dense Q5_K lm_head: logits[m][v] = half(W[v]·xh[m])   (head8 contract)."""
    return _k4_gemv("tlx_head8", 176, wq5, xh, logits, stream)


def _k4_dequant(name, nbytes, w, out, kdim, stream):
    rows = w.numel() // (nbytes * (kdim // 256))
    _need(out, rows * kdim * out.element_size(), "out")
    _dev(w, out)
    call(name, w.data_ptr(), out.data_ptr(), rows, kdim, int(out.dtype == _F16), _stream(stream))
    return out


def q4k_dequant(w, out, kdim, stream=None):
    return _k4_dequant("tlx_q4k_dequant", 144, w, out, kdim, stream)


def q5k_dequant(w, out, kdim, stream=None):
    return _k4_dequant("tlx_q5k_dequant", 176, w, out, kdim, stream)


def aq6k8(wq, wk, wv, gridf, xh, qrow, krow, vrow, layout=LAYOUT_PACKED, stream=None):
    """Fused attention projections with a Q6_K q (padded 212-B blocks for ``LAYOUT_PACKED``,
    raw 210-B for ``LAYOUT_RAW``), IQ3_XXS packed-row k, and v IQ3_XXS packed rows or (with
    ``V_Q4K`` in ``layout``) GGUF Q4_K."""
    base = layout & ~V_Q4K
    v = _q4k_rows if layout & V_Q4K else _iq3_rows
    _attn("tlx_aq6k8", wq, wk, wv, gridf, xh, qrow, krow, vrow,
          lambda n, k: _q6_rows(n, k, base), _iq3_rows, v, layout, stream)


# ------------------------------------------------------------------ prefill dequant-GEMMs
# Weights are IQ3_XXS in the packed7 unit layout (``formats.iq3_pack7``), as the reference's
# prefill GEMMs read them.
def pfg3_ffn(wg, wu, gridf, x16, out16, layout=LAYOUT_PACK7, stream=None):
    """out16[m] = silu16(half(Wg·x16[m])) * half(Wu·x16[m]) over a prompt chunk
    (pf_gemm3 FFN=1: kernel(w1, w2, gridf, x16, out16))."""
    M, K, N = x16.shape[0], x16.shape[1], out16.shape[1]
    _need(wg, _pack7(N, K), "wg (packed7)")
    _need(wu, _pack7(N, K), "wu (packed7)")
    _need(gridf, 4096, "gridf")
    _need(out16, M * N * 2, "out16")
    _dev(wg, wu, gridf, x16, out16)
    _ws(x16)
    call("tlx_pfg3_ffn", wg.data_ptr(), wu.data_ptr(), gridf.data_ptr(), x16.data_ptr(), out16.data_ptr(),
         M, N, K, layout, _stream(stream))
    return out16


# The merged form (pf_gemm3m): segments of different weight classes sharing x16, one launch.
_PFM_CLASSES = {   # (ggml type, layout) -> bytes of an n x k matrix
    (18, LAYOUT_PACK7): lambda n, k: _pack7(n, k),
    (12, LAYOUT_RAW): lambda n, k: n * 144 * (k // 256),
    (13, LAYOUT_RAW): lambda n, k: n * 176 * (k // 256),
    (14, LAYOUT_PACKED): lambda n, k: n * 212 * (k // 256),
}


def pfg3m(ws, outs, types, layouts, gridf, x16, stream=None):
    """outs[s][m] = half(W_s·x16[m]) for up to three matrices of different weight classes in one
    launch (pf_gemm3m: kernel(wA, wB[, wC], gridf, x16, outA, outB[, outC])).  types: ggml type codes
    (18 IQ3_XXS with LAYOUT_PACK7, 12 Q4_K / 13 Q5_K with LAYOUT_RAW, 14 Q6_K with LAYOUT_PACKED, the
    padded 212-B blocks)."""
    import ctypes
    nseg = len(ws)
    if not 1 <= nseg == len(outs) == len(types) == len(layouts) <= 3:
        raise ValueError("one to three segments: a weight, output, type and layout each")
    M, K = x16.shape
    for w, o, t, lay in zip(ws, outs, types, layouts):
        size = _PFM_CLASSES.get((int(t), int(lay)))
        if size is None:
            raise ValueError(f"weight class (type {t}, layout {lay}) is not a merged-GEMM segment class")
        _need(w, size(o.shape[-1], K), "w")
        _need(o, M * o.shape[-1] * 2, "out")
        _dev(w, o)
    _need(gridf, 4096, "gridf")
    _dev(gridf, x16)
    _ws(x16)
    P = ctypes.c_void_p * nseg
    I = ctypes.c_int * nseg
    call("tlx_pfg3m", P(*[w.data_ptr() for w in ws]), P(*[o.data_ptr() for o in outs]),
         I(*[o.shape[-1] for o in outs]), I(*[int(t) for t in types]), I(*[int(lay) for lay in layouts]), nseg,
         gridf.data_ptr(), x16.data_ptr(), M, K, _stream(stream))
    return outs


# ------------------------------------------------------------------ repackers (device to device)
def pack_iq3_rows(raw, packed, N, K, stream=None):
    """Raw IQ3_XXS rows [N][K/256][98 B] -> packed rows [qs][sw][d] (pack_w1c.pack_iq3)."""
    nbytes = N * 98 * (K // 256)
    _need(raw, nbytes, "raw")
    _need(packed, nbytes, "packed")
    _dev(raw, packed)
    call("tlx_pack_iq3_rows", raw.data_ptr(), packed.data_ptr(), N, K, _stream(stream))
    return packed


def pack_q6_pad(raw, padded, N, K, stream=None):
    """Raw Q6_K rows [N][K/256][210 B] -> padded 212-B blocks (pack_w1c.pack_q6)."""
    _need(raw, N * 210 * (K // 256), "raw")
    _need(padded, N * 212 * (K // 256), "padded")
    _dev(raw, padded)
    call("tlx_pack_q6_pad", raw.data_ptr(), padded.data_ptr(), N, K, _stream(stream))
    return padded


def pack_w7(packed, p7, N, K, stream=None):
    """Packed IQ3_XXS rows -> packed7 units [N/8][K/128][32][16 B] (pack_w7.pack_tensor)."""
    _need(packed, N * 98 * (K // 256), "packed")
    _need(p7, _pack7(N, K), "p7")
    _dev(packed, p7)
    call("tlx_pack_w7", packed.data_ptr(), p7.data_ptr(), N, K, _stream(stream))
    return p7


def pack_iq3_tiled(src, tiled, N, K, src_layout=LAYOUT_PACKED, stream=None):
    """IQ3_XXS rows (GGUF blocks or packed rows) -> the tile-major records the decode GEMVs read
    with ``layout=LAYOUT_TILED`` (ceil(N/16) * K/256 * 1632 B: the GGUF bytes re-encoded with the
    per-chunk table indices precomputed)."""
    _need(src, _iq3_rows(N, K), "src")
    _need(tiled, _iq3_w(N, K, LAYOUT_TILED), "tiled")
    _dev(src, tiled)
    call("tlx_pack_iq3_tiled", src.data_ptr(), tiled.data_ptr(), N, K, src_layout, _stream(stream))
    return tiled


def pack_iq4_tiled(src, tiled, N, K, stream=None):
    """IQ4_XS GGUF rows u8[N][K/256*136] -> the tiled records the MoE expert GEMMs read with
    ``layout=LAYOUT_TILED`` (same size: a byte permutation per 16-row tile and 256-k block)."""
    nbytes = N * (K // 256) * 136
    _need(src, nbytes, "src")
    _need(tiled, nbytes, "tiled")
    _dev(src, tiled)
    call("tlx_pack_iq4_tiled", src.data_ptr(), tiled.data_ptr(), N, K, _stream(stream))
    return tiled


def pack_iq3s_tiled(src, tiled, N, K, stream=None):
    """IQ3_S GGUF rows u8[N][K/256*110] -> the tiled records the checkpoint-class expert GEMMs read
    with ``layout=LAYOUT_TILED`` (same size: a byte permutation per 16-row tile and 256-k block)."""
    nbytes = N * (K // 256) * 110
    _need(src, nbytes, "src")
    _need(tiled, nbytes, "tiled")
    _dev(src, tiled)
    call("tlx_pack_iq3s_tiled", src.data_ptr(), tiled.data_ptr(), N, K, _stream(stream))
    return tiled


def pack_q6k_tiled(src, tiled, N, K, stream=None):
    """Q6_K GGUF rows u8[N][K/256*210] -> the tiled records of ``layout=LAYOUT_TILED`` (same size)."""
    nbytes = N * (K // 256) * 210
    _need(src, nbytes, "src")
    _need(tiled, nbytes, "tiled")
    _dev(src, tiled)
    call("tlx_pack_q6k_tiled", src.data_ptr(), tiled.data_ptr(), N, K, _stream(stream))
    return tiled


def p8_quant(x16, xq, sx, rs, stream=None):
    """Per (row, 128-k chunk) int8 quantization of fp16 activations (pfk_q8: kernel(x, xq, sx, rs))."""
    M, K = x16.shape
    if K % 128:
        raise ValueError("K must be a multiple of 128")
    _need(xq, M * K, "xq")
    _need(sx, M * (K // 128) * 4, "sx")
    _need(rs, M * (K // 128) * 4, "rs")
    _dev(x16, xq, sx, rs)
    call("tlx_p8_quant", x16.data_ptr(), xq.data_ptr(), sx.data_ptr(), rs.data_ptr(), M, K, _stream(stream))
    return xq, sx, rs


def p8w4_ffn(w1u, w2u, lut8, xq, sx, out16, layout=LAYOUT_PACK7, stream=None):
    """W4A8 gate+up + SwiGLU over int8 activations (p8w4ffn7: kernel(w1u, w2u, lut8, xq, sx, out16))."""
    M, K, N = xq.shape[0], xq.shape[1], out16.shape[1]
    _need(w1u, _pack7(N, K), "w1u (packed7)")
    _need(w2u, _pack7(N, K), "w2u (packed7)")
    _need(lut8, 1024, "lut8")
    _need(sx, M * (K // 128) * 4, "sx")
    _need(out16, M * N * 2, "out16")
    _dev(w1u, w2u, lut8, xq, sx, out16)
    call("tlx_p8w4_ffn", w1u.data_ptr(), w2u.data_ptr(), lut8.data_ptr(), xq.data_ptr(), sx.data_ptr(),
         out16.data_ptr(), M, N, K, layout, _stream(stream))
    return out16


def pfg3_iq3d(w, gridf, x16, res16, out32, layout=LAYOUT_PACK7, stream=None):
    """out32[m] = res16[m] + W·x16[m]   (pf_gemm3 RES=1: kernel(w1, gridf, x16, res16, out32))."""
    M, K, N = x16.shape[0], x16.shape[1], out32.shape[1]
    _need(w, _pack7(N, K), "w (packed7)")
    _need(gridf, 4096, "gridf")
    _need(res16, M * N * 4, "res16")
    _need(out32, M * N * 4, "out32")
    _dev(w, gridf, x16, res16, out32)
    _ws(x16)
    call("tlx_pfg3_iq3d", w.data_ptr(), gridf.data_ptr(), x16.data_ptr(), res16.data_ptr(), out32.data_ptr(),
         M, N, K, layout, _stream(stream))
    return out32


def pfg3_iq3o(w, gridf, x16, out16, layout=LAYOUT_PACK7, stream=None):
    """out16[m] = half(W·x16[m])   (pf_gemm3 plain: kernel(w1, gridf, x16, out16))."""
    M, K, N = x16.shape[0], x16.shape[1], out16.shape[1]
    _need(w, _pack7(N, K), "w (packed7)")
    _need(gridf, 4096, "gridf")
    _need(out16, M * N * 2, "out16")
    _dev(w, gridf, x16, out16)
    _ws(x16)
    call("tlx_pfg3_iq3o", w.data_ptr(), gridf.data_ptr(), x16.data_ptr(), out16.data_ptr(), M, N, K, layout,
         _stream(stream))
    return out16


# ------------------------------------------------------------------ MoE grouped experts
# 256 routed experts + 1 shared, hidden 2048, expert intermediate 512, top-8, IQ4_XS weights.
# ptbl / ptbl_dn: int64 device tensors of 256 slab addresses (formats.pointer_table).
def moe_topk(logits, eids, gates, stream=None):
    """Top-8 + renormalized softmax from router logits [P][256] (the rt8e256 epilogue)."""
    P = logits.shape[0]
    _need(logits, P * 256 * 4, "logits")
    _need(eids, P * 8 * 2, "eids")
    _need(gates, P * 8 * 4, "gates")
    _dev(logits, eids, gates)
    call("tlx_moe_topk", logits.data_ptr(), eids.data_ptr(), gates.data_ptr(), logits.shape[0], _stream(stream))


def moe_route(wrt, wsh, h, eids, gates, sg, stream=None):
    """rt8e256(wrt, wsh, h, eids, gates, sg)."""
    P = h.shape[0]
    _need(wrt, 256 * 2048 * 4, "wrt")
    _need(wsh, 2048 * 4, "wsh")
    _need(h, P * 2048 * 4, "h")
    _need(eids, P * 8 * 2, "eids")
    _need(gates, P * 8 * 4, "gates")
    _need(sg, P * 4, "sg")
    _dev(wrt, wsh, h, eids, gates, sg)
    call("tlx_moe_route", wrt.data_ptr(), wsh.data_ptr(), h.data_ptr(), eids.data_ptr(), gates.data_ptr(),
         sg.data_ptr(), h.shape[0], _stream(stream))


def moe_max_items(npair):
    from ._lib import lib
    return lib().tlx_moe_max_items(npair)


def moe_sort(eids, eoff, plist, items, nitp, stream=None):
    """mmsort8(eids, eoff, plist, items, nitp, np) with np = eids.numel()."""
    n = eids.numel()
    _need(eoff, 257 * 4, "eoff")
    _need(plist, n * 2, "plist")
    _need(items, moe_max_items(n) * 4, "items")
    _need(nitp, 4, "nitp")
    _dev(eids, eoff, plist, items, nitp)
    call("tlx_moe_sort", eids.data_ptr(), eoff.data_ptr(), plist.data_ptr(), items.data_ptr(), nitp.data_ptr(),
         eids.numel(), _stream(stream))


def moe_up4(ptbl, items, nitp, eoff, plist, xs, iq4nl, ys, stream=None, layout=LAYOUT_RAW):
    """gxm_up4(ptbl, items, nitp, eoff, plist, xs, iq4nlb, ys) over the sorted pairs:
    ys[pair][512] = silu(Wg_e . x[pos]) * (Wu_e . x[pos]), pos = pair >> 3.  layout: the slabs'
    (LAYOUT_RAW GGUF rows, LAYOUT_TILED records from ``pack_iq4_tiled``)."""
    n = ys.shape[0]
    _need(ptbl, 256 * 8, "ptbl")
    _need(eoff, 257 * 4, "eoff")
    _need(plist, n * 2, "plist")
    _need(items, moe_max_items(n) * 4, "items")
    _need(xs, (n // 8) * 2048 * 4, "xs")
    _need(ys, n * 512 * 4, "ys")
    _need(iq4nl, 64, "iq4nl")
    _dev(ptbl, eoff, plist, items, nitp, xs, iq4nl, ys)
    call("tlx_moe_up4", ptbl.data_ptr(), items.data_ptr(), nitp.data_ptr(), eoff.data_ptr(), plist.data_ptr(),
         xs.data_ptr(), iq4nl.data_ptr(), ys.data_ptr(), ys.shape[0], layout, _stream(stream))


def moe_dn4(ptbl_dn, items, nitp, eoff, plist, act, iq4nl, parts, stream=None, layout=LAYOUT_RAW):
    """gxm_dn(ptbl, items, nitp, eoff, plist, act, iq4nlb, parts) over the sorted pairs:
    parts[pair][2048] = fp16(Wd_e . act[pair])."""
    n = act.shape[0]
    _need(ptbl_dn, 256 * 8, "ptbl_dn")
    _need(eoff, 257 * 4, "eoff")
    _need(plist, n * 2, "plist")
    _need(items, moe_max_items(n) * 4, "items")
    _need(act, n * 512 * 4, "act")
    _need(parts, n * 2048 * 2, "parts")
    _need(iq4nl, 64, "iq4nl")
    _dev(ptbl_dn, eoff, plist, items, nitp, act, iq4nl, parts)
    call("tlx_moe_dn4", ptbl_dn.data_ptr(), items.data_ptr(), nitp.data_ptr(), eoff.data_ptr(), plist.data_ptr(),
         act.data_ptr(), iq4nl.data_ptr(), parts.data_ptr(), act.shape[0], layout, _stream(stream))


def moe_up4_pairs(ptbl, eids, xs, iq4nl, ys, stream=None, layout=LAYOUT_RAW):
    """gx8e256up4(ptbl, eids, xs, iq4nlb, ys): pair p runs expert eids[p] on x[p >> 3], no sort."""
    n = ys.shape[0]
    _need(ptbl, 256 * 8, "ptbl")
    _need(eids, n * 2, "eids")
    _need(xs, ((n + 7) // 8) * 2048 * 4, "xs")
    _need(ys, n * 512 * 4, "ys")
    _need(iq4nl, 64, "iq4nl")
    _dev(ptbl, eids, xs, iq4nl, ys)
    call("tlx_moe_up4_pairs", ptbl.data_ptr(), eids.data_ptr(), xs.data_ptr(), iq4nl.data_ptr(), ys.data_ptr(),
         n, layout, _stream(stream))


def moe_dn4_pairs(ptbl_dn, eids, act, iq4nl, parts, stream=None, layout=LAYOUT_RAW):
    """gx8e256dn(ptbl, eids, act, iq4nlb, parts): pair p runs expert eids[p] on act[p], no sort."""
    n = act.shape[0]
    _need(ptbl_dn, 256 * 8, "ptbl_dn")
    _need(eids, n * 2, "eids")
    _need(act, n * 512 * 4, "act")
    _need(parts, n * 2048 * 2, "parts")
    _need(iq4nl, 64, "iq4nl")
    _dev(ptbl_dn, eids, act, iq4nl, parts)
    call("tlx_moe_dn4_pairs", ptbl_dn.data_ptr(), eids.data_ptr(), act.data_ptr(), iq4nl.data_ptr(),
         parts.data_ptr(), n, layout, _stream(stream))


def moe_up4_pairs_sh(ptbl, eids, xs, iq4nl, ys, ptbl_sh, sact, stream=None, layout=LAYOUT_RAW):
    """moe_up4_pairs and the shared expert's gate+up (ptbl_sh[0] into sact [P][512]) in one
    launch; P = xs.shape[0], eids / ys over the 8 P pairs."""
    P = xs.shape[0]
    n = 8 * P
    _need(ptbl, 256 * 8, "ptbl")
    _need(ptbl_sh, 8, "ptbl_sh")
    _need(eids, n * 2, "eids")
    _need(xs, P * 2048 * 4, "xs")
    _need(ys, n * 512 * 4, "ys")
    _need(sact, P * 512 * 4, "sact")
    _need(iq4nl, 64, "iq4nl")
    _dev(ptbl, ptbl_sh, eids, xs, iq4nl, ys, sact)
    call("tlx_moe_up4_pairs_sh", ptbl.data_ptr(), eids.data_ptr(), xs.data_ptr(), iq4nl.data_ptr(), ys.data_ptr(),
         ptbl_sh.data_ptr(), sact.data_ptr(), P, layout, _stream(stream))


def moe_dn4_pairs_sh(ptbl_dn, eids, act, iq4nl, parts, ptbl_sh_dn, sact, shared, stream=None, layout=LAYOUT_RAW):
    """moe_dn4_pairs and the shared expert's down projection (ptbl_sh_dn[0], sact [P][512] into
    shared [P][2048] f32) in one launch; P = sact.shape[0], act / parts over the 8 P pairs."""
    P = sact.shape[0]
    n = 8 * P
    _need(ptbl_dn, 256 * 8, "ptbl_dn")
    _need(ptbl_sh_dn, 8, "ptbl_sh_dn")
    _need(eids, n * 2, "eids")
    _need(act, n * 512 * 4, "act")
    _need(parts, n * 2048 * 2, "parts")
    _need(sact, P * 512 * 4, "sact")
    _need(shared, P * 2048 * 4, "shared")
    _need(iq4nl, 64, "iq4nl")
    _dev(ptbl_dn, ptbl_sh_dn, eids, act, iq4nl, parts, sact, shared)
    call("tlx_moe_dn4_pairs_sh", ptbl_dn.data_ptr(), eids.data_ptr(), act.data_ptr(), iq4nl.data_ptr(),
         parts.data_ptr(), ptbl_sh_dn.data_ptr(), sact.data_ptr(), shared.data_ptr(), P, layout, _stream(stream))


def moe_up4_sh(ptbl, items, nitp, eoff, plist, xs, iq4nl, ys, ptbl_sh, sact, stream=None, layout=LAYOUT_RAW):
    """moe_up4 over the sorted pairs and the shared expert's gate+up (ptbl_sh[0] into sact
    [P][512], P = xs.shape[0]) in one launch where both run the MFMA forms (else the two
    launches); outputs those of moe_up4 and moe_shared's gate+up bit for bit."""
    n = ys.shape[0]
    P = xs.shape[0]
    _need(ptbl, 256 * 8, "ptbl")
    _need(ptbl_sh, 8, "ptbl_sh")
    _need(eoff, 257 * 4, "eoff")
    _need(plist, n * 2, "plist")
    _need(items, moe_max_items(n) * 4, "items")
    _need(xs, max(P, n // 8) * 2048 * 4, "xs")
    _need(ys, n * 512 * 4, "ys")
    _need(sact, P * 512 * 4, "sact")
    _need(iq4nl, 64, "iq4nl")
    _dev(ptbl, ptbl_sh, eoff, plist, items, nitp, xs, iq4nl, ys, sact)
    call("tlx_moe_up4_sh", ptbl.data_ptr(), items.data_ptr(), nitp.data_ptr(), eoff.data_ptr(), plist.data_ptr(),
         xs.data_ptr(), iq4nl.data_ptr(), ys.data_ptr(), n, ptbl_sh.data_ptr(), sact.data_ptr(), P, layout,
         _stream(stream))


def moe_dn4_sh(ptbl_dn, items, nitp, eoff, plist, act, iq4nl, parts, ptbl_sh_dn, sact, shared, stream=None,
               layout=LAYOUT_RAW):
    """moe_dn4 over the sorted pairs and the shared expert's down projection (ptbl_sh_dn[0],
    sact [P][512] into shared [P][2048] f32, P = sact.shape[0]) in one launch where both run the
    MFMA forms (else the two launches); outputs those of the separate calls bit for bit."""
    n = act.shape[0]
    P = sact.shape[0]
    _need(ptbl_dn, 256 * 8, "ptbl_dn")
    _need(ptbl_sh_dn, 8, "ptbl_sh_dn")
    _need(eoff, 257 * 4, "eoff")
    _need(plist, n * 2, "plist")
    _need(items, moe_max_items(n) * 4, "items")
    _need(act, n * 512 * 4, "act")
    _need(parts, n * 2048 * 2, "parts")
    _need(shared, P * 2048 * 4, "shared")
    _need(iq4nl, 64, "iq4nl")
    _dev(ptbl_dn, ptbl_sh_dn, eoff, plist, items, nitp, act, iq4nl, parts, sact, shared)
    call("tlx_moe_dn4_sh", ptbl_dn.data_ptr(), items.data_ptr(), nitp.data_ptr(), eoff.data_ptr(), plist.data_ptr(),
         act.data_ptr(), iq4nl.data_ptr(), parts.data_ptr(), n, ptbl_sh_dn.data_ptr(), sact.data_ptr(),
         shared.data_ptr(), P, layout, _stream(stream))


def moe_shared(ptbl_sh, xs, iq4nl, act, out, stream=None, layout=LAYOUT_RAW):
    """Shared expert over all positions: act [P][512] (scratch), out [P][2048] f32."""
    P = xs.shape[0]
    _need(ptbl_sh, 2 * 8, "ptbl_sh")
    _need(xs, P * 2048 * 4, "xs")
    _need(act, P * 512 * 4, "act")
    _need(out, P * 2048 * 4, "out")
    _need(iq4nl, 64, "iq4nl")
    _dev(ptbl_sh, xs, iq4nl, act, out)
    call("tlx_moe_shared", ptbl_sh.data_ptr(), xs.data_ptr(), iq4nl.data_ptr(), act.data_ptr(), out.data_ptr(),
         xs.shape[0], layout, _stream(stream))


def moe_combine(parts, gates, sg, shared, hres, y, stream=None):
    """cmbz2048(parts, gates, sg, shared, hres, y)."""
    P = y.shape[0]
    _need(parts, P * 8 * 2048 * 2, "parts")
    _need(gates, P * 8 * 4, "gates")
    _need(sg, P * 4, "sg")
    for t, nm in ((shared, "shared"), (hres, "hres"), (y, "y")):
        _need(t, P * 2048 * 4, nm)
    _dev(parts, gates, sg, shared, hres, y)
    call("tlx_moe_combine", parts.data_ptr(), gates.data_ptr(), sg.data_ptr(), shared.data_ptr(), hres.data_ptr(),
         y.data_ptr(), y.shape[0], _stream(stream))


# ---- the checkpoint's classes: IQ3_S routed gate/up, Q6_K routed down, Q8_0 shared expert
def moe_up3s(ptbl, eoff, plist, xs, gridf, ys, stream=None, layout=LAYOUT_RAW):
    """gxu_gm(ptbl, eoff, plist, xs, gridf, ys) over the sorted pairs (IQ3_S slabs: 512 gate rows
    then 512 up rows 450,560 B in, 880 B a row): ys[pair][512] = silu(Wg_e . x[pos]) * (Wu_e . x[pos]).
    ``layout=LAYOUT_TILED``: slabs repacked by pack_iq3s_tiled (same results bit for bit)."""
    n = ys.shape[0]
    _need(ptbl, 256 * 8, "ptbl")
    _need(eoff, 257 * 4, "eoff")
    _need(plist, n * 2, "plist")
    _need(xs, ((n + 7) // 8) * 2048 * 4, "xs")
    _need(ys, n * 512 * 4, "ys")
    _need(gridf, 512 * 16, "gridf")
    _dev(ptbl, eoff, plist, xs, gridf, ys)
    call("tlx_moe_up3s", ptbl.data_ptr(), eoff.data_ptr(), plist.data_ptr(), xs.data_ptr(), gridf.data_ptr(),
         ys.data_ptr(), n, layout, _stream(stream))


def moe_up3s_pairs(ptbl, eids, xs, gridf, ys, stream=None, layout=LAYOUT_RAW):
    """gx8e256up(ptbl, eids, xs, gridf, ys): pair p runs IQ3_S expert eids[p] on x[p >> 3], no sort."""
    n = ys.shape[0]
    _need(ptbl, 256 * 8, "ptbl")
    _need(eids, n * 2, "eids")
    _need(xs, ((n + 7) // 8) * 2048 * 4, "xs")
    _need(ys, n * 512 * 4, "ys")
    _need(gridf, 512 * 16, "gridf")
    _dev(ptbl, eids, xs, gridf, ys)
    call("tlx_moe_up3s_pairs", ptbl.data_ptr(), eids.data_ptr(), xs.data_ptr(), gridf.data_ptr(), ys.data_ptr(),
         n, layout, _stream(stream))


def moe_dn6(ptbl_dn, items, nitp, eoff, plist, act, parts, stream=None, layout=LAYOUT_RAW):
    """gxm_dn6(ptbl, items, nitp, eoff, plist, act, parts) over the sorted pairs (Q6_K slabs of
    2048 rows x 420 B): parts[pair][2048] = fp16(Wd_e . act[pair]).  ``layout=LAYOUT_TILED``: slabs
    repacked by pack_q6k_tiled."""
    n = act.shape[0]
    _need(ptbl_dn, 256 * 8, "ptbl_dn")
    _need(eoff, 257 * 4, "eoff")
    _need(plist, n * 2, "plist")
    _need(act, n * 512 * 4, "act")
    _need(parts, n * 2048 * 2, "parts")
    _dev(ptbl_dn, eoff, plist, act, parts)
    call("tlx_moe_dn6", ptbl_dn.data_ptr(), 0 if items is None else items.data_ptr(),
         0 if nitp is None else nitp.data_ptr(), eoff.data_ptr(), plist.data_ptr(), act.data_ptr(), parts.data_ptr(),
         n, layout, _stream(stream))


def moe_up3s_sh(ptbl, eoff, plist, xs, gridf, ys, wg8, wu8, sact, stream=None, layout=LAYOUT_RAW):
    """moe_up3s over the sorted pairs and the Q8_0 shared expert's gate+up (wg8 / wu8 rows, into
    sact [P][512], P = xs.shape[0]) in one launch above P = 16 (else the two launches); outputs
    those of moe_up3s and moe_shared8's gate+up bit for bit."""
    n = ys.shape[0]
    P = xs.shape[0]
    _need(ptbl, 256 * 8, "ptbl")
    _need(eoff, 257 * 4, "eoff")
    _need(plist, n * 2, "plist")
    _need(xs, max(P, (n + 7) // 8) * 2048 * 4, "xs")
    _need(ys, n * 512 * 4, "ys")
    _need(gridf, 512 * 16, "gridf")
    _need(wg8, 512 * 2176, "wg8")
    _need(wu8, 512 * 2176, "wu8")
    _need(sact, P * 512 * 4, "sact")
    _dev(ptbl, eoff, plist, xs, gridf, ys, wg8, wu8, sact)
    call("tlx_moe_up3s_sh", ptbl.data_ptr(), eoff.data_ptr(), plist.data_ptr(), xs.data_ptr(), gridf.data_ptr(),
         ys.data_ptr(), n, wg8.data_ptr(), wu8.data_ptr(), sact.data_ptr(), P, layout, _stream(stream))


def moe_dn6_sh(ptbl_dn, items, nitp, eoff, plist, act, parts, wd8, sact, shared, stream=None, layout=LAYOUT_RAW):
    """moe_dn6 over the sorted pairs and the Q8_0 shared expert's down projection (wd8 rows, sact
    [P][512] into shared [P][2048] f32, P = sact.shape[0]) in one launch above P = 16 (else the
    two launches); outputs those of the separate calls bit for bit."""
    n = act.shape[0]
    P = sact.shape[0]
    _need(ptbl_dn, 256 * 8, "ptbl_dn")
    _need(eoff, 257 * 4, "eoff")
    _need(plist, n * 2, "plist")
    _need(act, n * 512 * 4, "act")
    _need(parts, n * 2048 * 2, "parts")
    _need(wd8, 2048 * 544, "wd8")
    _need(shared, P * 2048 * 4, "shared")
    _dev(ptbl_dn, eoff, plist, act, parts, wd8, sact, shared)
    call("tlx_moe_dn6_sh", ptbl_dn.data_ptr(), None if items is None else items.data_ptr(),
         None if nitp is None else nitp.data_ptr(), eoff.data_ptr(), plist.data_ptr(), act.data_ptr(),
         parts.data_ptr(), n, wd8.data_ptr(), sact.data_ptr(), shared.data_ptr(), P, layout, _stream(stream))


def moe_dn6_pairs(ptbl_dn, eids, act, parts, stream=None, layout=LAYOUT_RAW):
    """gx8e256dn6(ptbl, eids, act, parts): pair p runs Q6_K expert eids[p] on act[p], no sort."""
    n = act.shape[0]
    _need(ptbl_dn, 256 * 8, "ptbl_dn")
    _need(eids, n * 2, "eids")
    _need(act, n * 512 * 4, "act")
    _need(parts, n * 2048 * 2, "parts")
    _dev(ptbl_dn, eids, act, parts)
    call("tlx_moe_dn6_pairs", ptbl_dn.data_ptr(), eids.data_ptr(), act.data_ptr(), parts.data_ptr(), n, layout,
         _stream(stream))


def moe_up3s_pairs_sh(ptbl, eids, xs, gridf, ys, wg8, wu8, sact, stream=None, layout=LAYOUT_RAW):
    """moe_up3s_pairs and the Q8_0 shared expert's gate+up (wg8 / wu8 rows, into sact [P][512],
    P = sact.shape[0]) in one launch at P <= 16 (else the two launches); outputs those of
    moe_up3s_pairs and moe_shared8's gate+up bit for bit."""
    n = ys.shape[0]
    P = sact.shape[0]
    _need(ptbl, 256 * 8, "ptbl")
    _need(eids, n * 2, "eids")
    _need(xs, max(P, (n + 7) // 8) * 2048 * 4, "xs")
    _need(ys, n * 512 * 4, "ys")
    _need(gridf, 512 * 16, "gridf")
    _need(wg8, 512 * 2176, "wg8")
    _need(wu8, 512 * 2176, "wu8")
    _need(sact, P * 512 * 4, "sact")
    _dev(ptbl, eids, xs, gridf, ys, wg8, wu8, sact)
    call("tlx_moe_up3s_pairs_sh", ptbl.data_ptr(), eids.data_ptr(), xs.data_ptr(), gridf.data_ptr(), ys.data_ptr(),
         n, wg8.data_ptr(), wu8.data_ptr(), sact.data_ptr(), P, layout, _stream(stream))


def moe_dn6_pairs_sh(ptbl_dn, eids, act, parts, wd8, sact, shared, stream=None, layout=LAYOUT_RAW):
    """moe_dn6_pairs and the Q8_0 shared expert's down projection (wd8 rows, sact [P][512] into
    shared [P][2048] f32) in one launch at P <= 16 (else the two launches); the separate calls' bits."""
    n = act.shape[0]
    P = sact.shape[0]
    _need(ptbl_dn, 256 * 8, "ptbl_dn")
    _need(eids, n * 2, "eids")
    _need(act, n * 512 * 4, "act")
    _need(parts, n * 2048 * 2, "parts")
    _need(wd8, 2048 * 544, "wd8")
    _need(shared, P * 2048 * 4, "shared")
    _dev(ptbl_dn, eids, act, parts, wd8, sact, shared)
    call("tlx_moe_dn6_pairs_sh", ptbl_dn.data_ptr(), eids.data_ptr(), act.data_ptr(), parts.data_ptr(), n,
         wd8.data_ptr(), sact.data_ptr(), shared.data_ptr(), P, layout, _stream(stream))


def moe_shared8(wg, wu, wd, x, y, act, stream=None):
    """shexp8(wg, wu, wd, x, y): the Q8_0 shared expert over P = x.shape[0] positions,
    y[P][2048] f32 = Wd . (silu(Wg . x) * (Wu . x)); act: caller scratch f32 [P][512]."""
    P = x.shape[0]
    _need(wg, 512 * 2176, "wg")
    _need(wu, 512 * 2176, "wu")
    _need(wd, 2048 * 544, "wd")
    _need(x, P * 2048 * 4, "x")
    _need(y, P * 2048 * 4, "y")
    _need(act, P * 512 * 4, "act")
    _dev(wg, wu, wd, x, y, act)
    call("tlx_moe_shared8", wg.data_ptr(), wu.data_ptr(), wd.data_ptr(), x.data_ptr(), y.data_ptr(), act.data_ptr(),
         P, _stream(stream))


class MoeScratch:
    """Per-call buffers of one MoE layer over P positions (allocated once, like the reference's
    Bufs): router ids / gates, the sort's bins and items, routed and shared activations, parts."""

    def __init__(self, P, device="cuda"):
        np_ = 8 * P
        self.P = P
        self.eids = torch.empty(P, 8, dtype=torch.int16, device=device)
        self.gates = torch.empty(P, 8, dtype=torch.float32, device=device)
        self.eoff = torch.empty(257, dtype=torch.int32, device=device)
        self.plist = torch.empty(np_, dtype=torch.int16, device=device)
        self.items = torch.empty(moe_max_items(np_), dtype=torch.int32, device=device)
        self.nitp = torch.empty(1, dtype=torch.int32, device=device)
        self.act = torch.empty(np_, 512, dtype=torch.float32, device=device)
        self.parts = torch.empty(np_, 2048, dtype=torch.float16, device=device)
        self.sact = torch.empty(P, 512, dtype=torch.float32, device=device)
        self.shared = torch.empty(P, 2048, dtype=torch.float32, device=device)


_SIDE_STREAMS = {}

# Largest batch the MoE layer routes with the pair-walk forms by default: up to here the sort
# launch it skips costs more than the expert slabs that two pairs of the batch share and the
# pair walk reads twice.
MOE_PAIR_WALK_MAX_P = 16


def moe_layer(logits, sg, xs, hres, y, ptbl, ptbl_dn, ptbl_sh, iq4nl, scratch, stream=None, overlap_shared=None,
              layout=LAYOUT_RAW, pair_walk=None):
    """One MoE layer, the sequence of build_seq7 (engine/mm/MM_P7_lib.py:449-511): top-8 from
    the router logits, then either the grouped path (sort, grouped gate+up, grouped down:
    the reference's prefill sequence, :451-499) or the pair walk (gate+up and down per pair on
    the router's ids, no sort: its decode sequence, :501-507), the shared expert, and the
    combine into y.  Both give the same bits.  pair_walk None picks the pair walk for
    P <= MOE_PAIR_WALK_MAX_P.  By default the shared expert rides in the routed launches (the pair
    walk's: moe_up4_pairs_sh / moe_dn4_pairs_sh; the grouped forms': moe_up4_sh / moe_dn4_sh),
    where it fills the routed grids' last rounds.  With overlap_shared it runs on a second stream
    instead, joined before the combine (it needs neither the routing nor the routed experts);
    the results are the same bits.  Measured in graph replays: the second stream is slower on
    both paths -- a replay runs the captured branch on the same queue, after the routed kernels
    (P=2048: 253 vs 271 us), and its fork and join cost a decode-size replay 4-10 us.  layout:
    the expert slabs' (all of them, shared expert included)."""
    sc = scratch
    if pair_walk is None:
        pair_walk = xs.shape[0] <= MOE_PAIR_WALK_MAX_P
    if overlap_shared is None:
        overlap_shared = False
    cur = stream if isinstance(stream, torch.cuda.Stream) else torch.cuda.current_stream()
    side = None
    if overlap_shared:
        side = _SIDE_STREAMS.get(cur.device)
        if side is None:
            side = _SIDE_STREAMS[cur.device] = torch.cuda.Stream(device=cur.device)
        side.wait_stream(cur)
        moe_shared(ptbl_sh, xs, iq4nl, sc.sact, sc.shared, stream=side, layout=layout)
    moe_topk(logits, sc.eids, sc.gates, stream=cur)
    if pair_walk and side is None:   # the shared expert rides in the pair walk's launches
        eids = sc.eids.view(-1)
        moe_up4_pairs_sh(ptbl, eids, xs, iq4nl, sc.act, ptbl_sh[0:1], sc.sact, stream=cur, layout=layout)
        moe_dn4_pairs_sh(ptbl_dn, eids, sc.act, iq4nl, sc.parts, ptbl_sh[1:2], sc.sact, sc.shared, stream=cur,
                         layout=layout)
        moe_combine(sc.parts, sc.gates, sg, sc.shared, hres, y, stream=cur)
        return y
    if pair_walk:
        eids = sc.eids.view(-1)
        moe_up4_pairs(ptbl, eids, xs, iq4nl, sc.act, stream=cur, layout=layout)
        moe_dn4_pairs(ptbl_dn, eids, sc.act, iq4nl, sc.parts, stream=cur, layout=layout)
    else:
        moe_sort(sc.eids, sc.eoff, sc.plist, sc.items, sc.nitp, stream=cur)
        if side is None:   # the shared expert rides in the grouped launches
            moe_up4_sh(ptbl, sc.items, sc.nitp, sc.eoff, sc.plist, xs, iq4nl, sc.act, ptbl_sh[0:1], sc.sact,
                       stream=cur, layout=layout)
            moe_dn4_sh(ptbl_dn, sc.items, sc.nitp, sc.eoff, sc.plist, sc.act, iq4nl, sc.parts, ptbl_sh[1:2],
                       sc.sact, sc.shared, stream=cur, layout=layout)
        else:
            moe_up4(ptbl, sc.items, sc.nitp, sc.eoff, sc.plist, xs, iq4nl, sc.act, stream=cur, layout=layout)
            moe_dn4(ptbl_dn, sc.items, sc.nitp, sc.eoff, sc.plist, sc.act, iq4nl, sc.parts, stream=cur,
                    layout=layout)
    if side is not None:
        cur.wait_stream(side)
    moe_combine(sc.parts, sc.gates, sg, sc.shared, hres, y, stream=cur)
    return y


def moe_layer_ckpt(logits, sg, xs, hres, y, ptbl, ptbl_dn, shared8, gridf, scratch, stream=None, down="q6k",
                   iq4nl=None, pair_walk=None, overlap_shared=None, layout=LAYOUT_RAW):
    """One MoE layer with the reference checkpoint's classes, the same sequence as moe_layer:
    top-8, then the pair walk (P <= MOE_PAIR_WALK_MAX_P by default) or sort + grouped forms for
    the IQ3_S gate+up, the down projection -- ``down`` "q6k" (Q6_K slabs, the checkpoint's layers
    34/38/39) or "iq4" (IQ4_XS GGUF-row slabs, iq4nl given) -- the Q8_0 shared expert
    (shared8 = (wg, wu, wd) rows), and the combine into y.  overlap_shared as moe_layer's: by
    default the shared expert rides in the routed launches (the pair walk's moe_up3s_pairs_sh /
    moe_dn6_pairs_sh, the grouped forms' moe_up3s_sh / moe_dn6_sh); with it, on a second stream
    joined before the combine.  ``layout`` (LAYOUT_RAW or LAYOUT_TILED) is that of the routed
    slabs, gate/up and down alike (pack_iq3s_tiled, pack_q6k_tiled / pack_iq4_tiled)."""
    sc = scratch
    if pair_walk is None:
        pair_walk = xs.shape[0] <= MOE_PAIR_WALK_MAX_P
    if overlap_shared is None:
        overlap_shared = False
    cur = stream if isinstance(stream, torch.cuda.Stream) else torch.cuda.current_stream()
    side = None
    if overlap_shared:
        side = _SIDE_STREAMS.get(cur.device)
        if side is None:
            side = _SIDE_STREAMS[cur.device] = torch.cuda.Stream(device=cur.device)
        side.wait_stream(cur)
        moe_shared8(*shared8, xs, sc.shared, sc.sact, stream=side)
    moe_topk(logits, sc.eids, sc.gates, stream=cur)
    eids = sc.eids.view(-1)
    wg8, wu8, wd8 = shared8
    # the shared expert in the routed launches (the Q6_K down layers; with an IQ4_XS down the
    # shared expert keeps its own two launches)
    fused = side is None and down == "q6k"
    if pair_walk:
        if fused:
            moe_up3s_pairs_sh(ptbl, eids, xs, gridf, sc.act, wg8, wu8, sc.sact, stream=cur, layout=layout)
            moe_dn6_pairs_sh(ptbl_dn, eids, sc.act, sc.parts, wd8, sc.sact, sc.shared, stream=cur, layout=layout)
        else:
            moe_up3s_pairs(ptbl, eids, xs, gridf, sc.act, stream=cur, layout=layout)
            if down == "q6k":
                moe_dn6_pairs(ptbl_dn, eids, sc.act, sc.parts, stream=cur, layout=layout)
            else:
                moe_dn4_pairs(ptbl_dn, eids, sc.act, iq4nl, sc.parts, stream=cur, layout=layout)
    else:
        moe_sort(sc.eids, sc.eoff, sc.plist, sc.items, sc.nitp, stream=cur)
        if fused:
            moe_up3s_sh(ptbl, sc.eoff, sc.plist, xs, gridf, sc.act, wg8, wu8, sc.sact, stream=cur, layout=layout)
        else:
            moe_up3s(ptbl, sc.eoff, sc.plist, xs, gridf, sc.act, stream=cur, layout=layout)
        if fused:
            moe_dn6_sh(ptbl_dn, sc.items, sc.nitp, sc.eoff, sc.plist, sc.act, sc.parts, wd8, sc.sact, sc.shared,
                       stream=cur, layout=layout)
        elif down == "q6k":
            moe_dn6(ptbl_dn, sc.items, sc.nitp, sc.eoff, sc.plist, sc.act, sc.parts, stream=cur, layout=layout)
        else:
            moe_dn4(ptbl_dn, sc.items, sc.nitp, sc.eoff, sc.plist, sc.act, iq4nl, sc.parts, stream=cur,
                    layout=layout)
    if side is not None:
        cur.wait_stream(side)
    elif not fused:
        moe_shared8(*shared8, xs, sc.shared, sc.sact, stream=cur)
    moe_combine(sc.parts, sc.gates, sg, sc.shared, hres, y, stream=cur)
    return y


# ------------------------------------------------------------------ measurement
def stream_read(src, sink, stream=None):
    """Read all of ``src`` once (HBM read-stream probe); ``sink`` receives one uint32 per wave.
    src's byte size must be a multiple of ``stream_chunk_bytes()``."""
    from ._lib import lib
    nbytes = src.numel() * src.element_size()
    chunk = lib().tlx_stream_chunk_bytes()
    _need(sink, 4 * 4 * (nbytes // chunk), "sink")
    _dev(src, sink)
    call("tlx_stream_read", src.data_ptr(), nbytes, sink.data_ptr(), _stream(stream))
    return sink


def stream_chunk_bytes():
    from ._lib import lib
    return lib().tlx_stream_chunk_bytes()
