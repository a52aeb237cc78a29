"""Decode GEMVs over the packed7 plane (TLX_LAYOUT_PACK7), the prefill GEMM's weight layout.

The reference's PF_DR7 mode uploads the FFN weights once, as packed7, and runs its decode
GEMVs on that plane (ffn8r7 / ffn8v{3,8,11}r7 / down8r7 / down8nw32v{3,8,11}r7,
/root/reference/engine/trunk_w1c.py:20-25,88-93, engine/ffn8v11r7.cu:4-16): "bit-identical by
construction" to the packed-row kernels, only the addressing changes.  Checked here the same
way: the packed7 GEMVs against the oracle (rel-err <= 1e-3 per row), bit for bit against the
packed-row GEMVs on the same weights, rows of an M-wide call bit-identical to M=1 calls, and
the prefill GEMM and the decode GEMV reading one and the same device buffer.
"""
import numpy as np
import pytest
import torch

from oracle import gemv, layouts, quants
from thunderllamax_amd import formats, ops, synth
from thunderllamax_amd._lib import LAYOUT_PACK7, LAYOUT_PACKED, LAYOUT_RAW, TlxError

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _planes(rng, rows, kdim, dev):
    raw = synth.iq3xxs_raw(rng, rows, kdim)
    packed = formats.iq3_pack_rows(raw, kdim)
    p7 = layouts.pack_w7(packed, kdim)        # the oracle's restatement of pack_w7.py
    assert np.array_equal(p7, formats.iq3_pack7(packed, kdim))
    return packed, torch.from_numpy(packed).to(dev), torch.from_numpy(np.ascontiguousarray(p7)).to(dev)


def _rows_err(y, ref):
    return max(gemv.rel_err(y[m], ref[m]) for m in range(ref.shape[0]))


def _bits(t):
    return t.view(torch.int16) if t.dtype == torch.float16 else t.view(torch.int32)


@pytest.mark.parametrize("M", [1, 4, 8, 11])
def test_ffn8_pack7_parity_and_bits(gpu, M):
    print(f"[case] ffn8 pack7 M={M} N=512 K=5120", flush=True)
    rng = np.random.default_rng(700 + M)
    N, K = 512, 5120
    pg, wg, wg7 = _planes(rng, N, K, gpu)
    pu, wu, wu7 = _planes(rng, N, K, gpu)
    x = torch.from_numpy(synth.activations_f16(rng, M, K)).to(gpu)
    g = formats.gridf_tensor(gpu)
    o7 = torch.empty(M, N, dtype=torch.float16, device=gpu)
    op = torch.empty_like(o7)
    ops.ffn8(wg7, wu7, g, x, o7, LAYOUT_PACK7)
    ops.ffn8(wg, wu, g, x, op, LAYOUT_PACKED)
    torch.cuda.synchronize()
    assert torch.equal(_bits(o7), _bits(op))
    _, _, ref = gemv.ffn8_ref(quants.dequant_iq3xxs_packed(pg, K), quants.dequant_iq3xxs_packed(pu, K),
                              x.cpu().numpy())
    err = _rows_err(o7.cpu().numpy(), ref)
    print(f"[ffn8 pack7 M={M}] max row rel-err {err:.3e}")
    assert err <= TOL


def test_ffn8_pack7_full_size_m11(gpu):
    """Config 2 (N = 17408, K = 5120) at M = 11: every row bit-identical to the packed-row GEMV,
    384 seeded rows against the oracle, and rows of the M = 11 call equal to M = 1 calls."""
    print("[case] ffn8 pack7 full-size M=11", flush=True)
    rng = synth.config_rng(2)
    N, K, M = 17408, 5120, 11
    pg, wg, wg7 = _planes(rng, N, K, gpu)
    pu, wu, wu7 = _planes(rng, N, K, gpu)
    xn = synth.activations_f16(rng, M, K)
    x = torch.from_numpy(xn).to(gpu)
    g = formats.gridf_tensor(gpu)
    o7 = torch.empty(M, N, dtype=torch.float16, device=gpu)
    op = torch.empty_like(o7)
    ops.ffn8(wg7, wu7, g, x, o7, LAYOUT_PACK7)
    ops.ffn8(wg, wu, g, x, op, LAYOUT_PACKED)
    one = torch.empty(1, N, dtype=torch.float16, device=gpu)
    for r in (0, 5, 10):
        ops.ffn8(wg7, wu7, g, x[r:r + 1].contiguous(), one, LAYOUT_PACK7)
        assert torch.equal(_bits(one[0]), _bits(o7[r])), r
    torch.cuda.synchronize()
    assert torch.equal(_bits(o7), _bits(op))
    rows = np.sort(np.random.default_rng(3).choice(N, 384, replace=False))
    _, _, ref = gemv.ffn8_ref(quants.dequant_iq3xxs_packed(pg[rows], K), quants.dequant_iq3xxs_packed(pu[rows], K), xn)
    err = _rows_err(o7.cpu().numpy()[:, rows], ref)
    print(f"[ffn8 pack7 full] sampled max row rel-err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("M", [1, 4, 8, 11])
def test_down8_pack7_parity_and_bits(gpu, M):
    print(f"[case] down8 pack7 M={M} N=5120 K=17408", flush=True)
    rng = np.random.default_rng(710 + M)
    N, K = 5120, 17408
    pd, wd, wd7 = _planes(rng, N, K, gpu)
    gn = synth.activations_f16(rng, M, K)
    hh = rng.standard_normal((M, N)).astype(np.float32)
    gact, hht = torch.from_numpy(gn).to(gpu), torch.from_numpy(hh).to(gpu)
    g = formats.gridf_tensor(gpu)
    y7 = torch.empty(M, N, dtype=torch.float32, device=gpu)
    yp = torch.empty_like(y7)
    ops.down8(wd7, g, gact, hht, y7, LAYOUT_PACK7)
    ops.down8(wd, g, gact, hht, yp, LAYOUT_PACKED)
    torch.cuda.synchronize()
    assert torch.equal(_bits(y7), _bits(yp))
    rows = np.sort(np.random.default_rng(4).choice(N, 256, replace=False))
    _, ref = gemv.down8_ref(quants.dequant_iq3xxs_packed(pd[rows], K), gn, hh[:, rows])
    err = _rows_err(y7.cpu().numpy()[:, rows] - hh[:, rows], ref - hh[:, rows])
    print(f"[down8 pack7 M={M}] sampled max row rel-err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("N", [8, 24, 1000])
def test_iq3_gemv_pack7_odd_tiles(gpu, N):
    """N % 16 == 8 leaves a half tile (one 8-row group): loads clamp, stores mask."""
    print(f"[case] iq3_gemv pack7 N={N}", flush=True)
    rng = np.random.default_rng(720 + N)
    K, M = 512, 3
    pw, w, w7 = _planes(rng, N, K, gpu)
    xn = synth.activations_f16(rng, M, K)
    x = torch.from_numpy(xn).to(gpu)
    g = formats.gridf_tensor(gpu)
    o7 = torch.empty(M, N, dtype=torch.float16, device=gpu)
    op = torch.empty_like(o7)
    ops.iq3_gemv(w7, g, x, o7, LAYOUT_PACK7)
    ops.iq3_gemv(w, g, x, op, LAYOUT_PACKED)
    torch.cuda.synchronize()
    assert torch.equal(_bits(o7), _bits(op))
    _, ref = gemv.gemv16_ref(quants.dequant_iq3xxs_packed(pw, K), xn)
    assert _rows_err(o7.cpu().numpy(), ref) <= TOL


def test_pack7_shared_plane_prefill_and_decode(gpu):
    """One packed7 buffer feeds the prefill GEMM (tlx_pfg3_ffn) and the decode GEMV (tlx_ffn8):
    both match the oracle on the same weights."""
    print("[case] pack7 shared plane", flush=True)
    rng = np.random.default_rng(730)
    N, K, Mp, Md = 256, 1024, 256, 11
    pg, _, wg7 = _planes(rng, N, K, gpu)
    pu, _, wu7 = _planes(rng, N, K, gpu)
    g = formats.gridf_tensor(gpu)
    Wg, Wu = quants.dequant_iq3xxs_packed(pg, K), quants.dequant_iq3xxs_packed(pu, K)
    xp = synth.activations_f16(rng, Mp, K)
    outp = torch.empty(Mp, N, dtype=torch.float16, device=gpu)
    ops.pfg3_ffn(wg7, wu7, g, torch.from_numpy(xp).to(gpu), outp)
    xd = synth.activations_f16(rng, Md, K)
    outd = torch.empty(Md, N, dtype=torch.float16, device=gpu)
    ops.ffn8(wg7, wu7, g, torch.from_numpy(xd).to(gpu), outd, LAYOUT_PACK7)
    torch.cuda.synchronize()
    assert _rows_err(outp.cpu().numpy()[:32], gemv.pf_ffn_ref(Wg, Wu, xp[:32])[2]) <= TOL
    assert _rows_err(outd.cpu().numpy(), gemv.ffn8_ref(Wg, Wu, xd)[2]) <= TOL


def _tileord(x):
    """Row-major [M][K] -> the tile-ordered copy [K/8][16][8] (slot r = row min(r, M - 1))."""
    M, K = x.shape
    idx = torch.clamp(torch.arange(16, device=x.device), max=M - 1)
    return x[idx].reshape(16, K // 8, 8).permute(1, 0, 2).contiguous()


@pytest.mark.parametrize("layout", [LAYOUT_PACKED, LAYOUT_RAW, LAYOUT_PACK7])
@pytest.mark.parametrize("M", [1, 5, 11])
def test_in_tileord_on_row_layouts(gpu, layout, M):
    """Tile-ordered activations give the row-major results bit for bit on the packed-row
    kernel's layouts too (ffn8, down8, plain)."""
    print(f"[case] in_tileord layout={layout} M={M}", flush=True)
    rng = np.random.default_rng(740 + M)
    N, K = 256, 2048
    raw = synth.iq3xxs_raw(rng, N, K)
    packed = formats.iq3_pack_rows(raw, K)
    src = {LAYOUT_PACKED: packed, LAYOUT_RAW: raw, LAYOUT_PACK7: formats.iq3_pack7(packed, K)}[layout]
    w = torch.from_numpy(np.ascontiguousarray(src)).to(gpu)
    g = formats.gridf_tensor(gpu)
    x = torch.from_numpy(synth.activations_f16(rng, M, K)).to(gpu)
    xt = _tileord(x)
    a = torch.empty(M, N, dtype=torch.float16, device=gpu)
    b = torch.empty_like(a)
    ops.ffn8(w, w, g, x, a, layout)
    ops.ffn8(w, w, g, xt, b, layout, in_tileord=True)
    hh = torch.zeros(M, N, dtype=torch.float32, device=gpu)
    ya, yb = torch.empty(M, N, dtype=torch.float32, device=gpu), torch.empty(M, N, dtype=torch.float32, device=gpu)
    ops.down8(w, g, x, hh, ya, layout)
    ops.down8(w, g, xt, hh, yb, layout, in_tileord=True)
    pa, pb = torch.empty_like(a), torch.empty_like(a)
    ops.iq3_gemv(w, g, x, pa, layout)
    ops.iq3_gemv(w, g, xt, pb, layout, in_tileord=True, m=M)
    torch.cuda.synchronize()
    assert torch.equal(_bits(a), _bits(b))
    assert torch.equal(_bits(ya), _bits(yb))
    assert torch.equal(_bits(pa), _bits(pb))


def test_pack7_rejects_bad_shapes(gpu):
    g = formats.gridf_tensor(gpu)
    w = torch.zeros(12 * 256, dtype=torch.uint8, device=gpu)
    x = torch.zeros(1, 256, dtype=torch.float16, device=gpu)
    with pytest.raises(TlxError):   # N % 8 != 0
        ops.iq3_gemv(w, g, x, torch.empty(1, 12, dtype=torch.float16, device=gpu), LAYOUT_PACK7)
    with pytest.raises(TlxError):   # 16-B alignment of the units
        ops.iq3_gemv(w[8:], g, x, torch.empty(1, 8, dtype=torch.float16, device=gpu), LAYOUT_PACK7)
