"""The tile-major records of the IQ3_XXS decode GEMVs (TLX_LAYOUT_TILED) and the balanced GEMV
kernel that reads them.

* The device repacker is byte-identical to the oracle's restatement (oracle/layouts.py
  ``pack_tiled``), from GGUF blocks and from packed rows, tail tiles included.
* Every GEMV entry point over the records stays within the path's rel-err 1e-3 of the oracle
  (exact product of the dequantized weights and the fp16 activations, then the epilogue), on
  shapes where tiles are split between waves of one workgroup and between two workgroups.
* Rows of an M-row call are bit-identical to M=1 calls, and repeated calls agree bit for bit
  (the cross-workgroup combine is ordered, not first-come).
"""
import numpy as np
import pytest
import torch

from oracle import gemv, layouts, quants
from thunderllamax_amd import formats, ops, synth
from thunderllamax_amd._lib import LAYOUT_PACKED, LAYOUT_RAW, LAYOUT_TILED, TlxError

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _tiled(gpu, src, N, K, src_layout=None):
    out = torch.empty(-(-N // 16) * 16 * 102 * (K // 256), dtype=torch.uint8, device=gpu)
    if src_layout is None:
        ops.pack_iq3_tiled(src, out, N, K)
    else:
        ops.pack_iq3_tiled(src, out, N, K, src_layout)
    return out


def _mat(gpu, rng, N, K):
    packed = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, N, K), K)
    return packed, _tiled(gpu, torch.from_numpy(packed).to(gpu), N, K)


def _rows_err(y, ref):
    return max(gemv.rel_err(y[m], ref[m]) for m in range(ref.shape[0]))


@pytest.mark.parametrize("N,K", [(16, 256), (37, 512), (64, 5120), (24, 17408)])
def test_pack_tiled_bytes(gpu, N, K):
    print(f"[case] pack_iq3_tiled N={N} K={K}", flush=True)
    raw = synth.iq3xxs_raw(synth.config_rng(5), N, K)
    packed = formats.iq3_pack_rows(raw, K)
    ref = layouts.pack_tiled(packed, K).reshape(-1)
    from_packed = _tiled(gpu, torch.from_numpy(packed).to(gpu), N, K)
    from_raw = _tiled(gpu, torch.from_numpy(raw.reshape(-1)).to(gpu), N, K, LAYOUT_RAW)
    torch.cuda.synchronize()
    assert np.array_equal(from_packed.cpu().numpy(), ref)
    assert np.array_equal(from_raw.cpu().numpy(), ref)


@pytest.mark.parametrize("M", [1, 4, 5, 6, 8, 11, 16])
def test_ffn8_tiled_parity(gpu, M):
    print(f"[case] ffn8 tiled M={M} N=1000 K=5120", flush=True)
    rng = synth.config_rng(2)
    N, K = 1000, 5120                       # 62.5 tiles: the tail tile has 8 zero rows
    pg, tg = _mat(gpu, rng, N, K)
    pu, tu = _mat(gpu, rng, N, K)
    x = synth.activations_f16(rng, M, K)
    out = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
    ops.ffn8(tg, tu, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), out, layout=LAYOUT_TILED)
    torch.cuda.synchronize()
    _, _, ref = gemv.ffn8_ref(quants.dequant_iq3xxs_packed(pg, K), quants.dequant_iq3xxs_packed(pu, K), x)
    err = _rows_err(out.cpu().numpy(), ref)
    print(f"[ffn8 tiled M={M}] max row rel-err {err:.3e}")
    assert err <= TOL


def test_ffn8_tiled_full_size(gpu):
    """Config 2 (N=17408, K=5120): tiles split between waves and between workgroups.  384 seeded
    rows against the oracle at M=11; every row of the M=11 call equals an M=1 call on that
    activation row bit for bit; two calls agree bit for bit."""
    print("[case] ffn8 tiled full-size", flush=True)
    rng = synth.config_rng(2)
    N, K, M = 17408, 5120, 11
    pg, tg = _mat(gpu, rng, N, K)
    pu, tu = _mat(gpu, rng, N, K)
    x = torch.from_numpy(synth.activations_f16(rng, M, K)).to(gpu)
    g = formats.gridf_tensor(gpu)
    full = torch.empty(M, N, dtype=torch.float16, device=gpu)
    again = torch.empty_like(full)
    ops.ffn8(tg, tu, g, x, full, layout=LAYOUT_TILED)
    ops.ffn8(tg, tu, g, x, again, layout=LAYOUT_TILED)
    one = torch.empty(M, N, dtype=torch.float16, device=gpu)
    for m in range(M):
        ops.ffn8(tg, tu, g, x[m:m + 1].contiguous(), one[m:m + 1], layout=LAYOUT_TILED)
    torch.cuda.synchronize()
    assert torch.equal(full.view(torch.int16), again.view(torch.int16))
    assert torch.equal(full.view(torch.int16), one.view(torch.int16))
    # every row (tiles shared between workgroups included) against the packed-row kernel, which
    # sums the same block products in another order
    ref_all = torch.empty_like(full)
    ops.ffn8(torch.from_numpy(pg).to(gpu), torch.from_numpy(pu).to(gpu), g, x, ref_all)
    torch.cuda.synchronize()
    d = (full.float() - ref_all.float()).abs()
    assert torch.isfinite(full.float()).all()
    assert (d <= 2e-3 * ref_all.float().abs() + 1e-3).all(), float(d.max())
    rows = np.sort(np.random.default_rng(1).choice(N, 384, replace=False))
    _, _, ref = gemv.ffn8_ref(quants.dequant_iq3xxs_packed(pg[rows], K),
                              quants.dequant_iq3xxs_packed(pu[rows], K), x.cpu().numpy())
    err = _rows_err(full.cpu().numpy()[:, rows], ref)
    print(f"[ffn8 tiled full] sampled max row rel-err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("M,N", [(1, 200), (11, 200), (11, 5120)])
def test_down8_and_plain_tiled_parity(gpu, M, N):
    print(f"[case] down8 / iq3_gemv tiled M={M} N={N} K=17408", flush=True)
    rng = synth.config_rng(3)
    K = 17408
    pd, td = _mat(gpu, rng, N, K)
    g = formats.gridf_tensor(gpu)
    x = synth.activations_f16(rng, M, K)
    hh = rng.standard_normal((M, N)).astype(np.float32)
    y = torch.empty(M, N, device=gpu)
    o = torch.empty(M, N, dtype=torch.float16, device=gpu)
    xd = torch.from_numpy(x).to(gpu)
    ops.down8(td, g, xd, torch.from_numpy(hh).to(gpu), y, layout=LAYOUT_TILED)
    ops.iq3_gemv(td, g, xd, o, layout=LAYOUT_TILED)
    torch.cuda.synchronize()
    rows = np.arange(N) if N <= 512 else np.sort(np.random.default_rng(2).choice(N, 256, replace=False))
    W = quants.dequant_iq3xxs_packed(pd[rows], K)
    _, yref = gemv.down8_ref(W, x, hh[:, rows])
    _, oref = gemv.gemv16_ref(W, x)
    ey = _rows_err(y.cpu().numpy()[:, rows], yref)
    eo = _rows_err(o.cpu().numpy()[:, rows], oref)
    print(f"[down8 tiled M={M} N={N}] rel-err {ey:.3e}; [iq3_gemv] {eo:.3e}")
    assert ey <= TOL and eo <= TOL


def test_odd_tile_count_parity(gpu):
    """A matrix of 513 tiles, the last one half full, alone (fp16 out and the residual form) and
    as the first of four matrices sharing x in one launch, against the oracle."""
    print("[case] odd tile count N=8200 K=512 M=5", flush=True)
    rng = synth.config_rng(9)
    M, K, ns = 5, 512, (8200, 600, 48, 40)
    packed = [formats.iq3_pack_rows(synth.iq3xxs_raw(rng, n, K), K) for n in ns]
    ws = [_tiled(gpu, torch.from_numpy(p).to(gpu), n, K) for p, n in zip(packed, ns)]
    g = formats.gridf_tensor(gpu)
    x = synth.activations_f16(rng, M, K)
    xd = torch.from_numpy(x).to(gpu)
    N0 = ns[0]
    hh = rng.standard_normal((M, N0)).astype(np.float32)
    y = torch.empty(M, N0, device=gpu)
    o = torch.full((M, N0), float("nan"), dtype=torch.float16, device=gpu)
    ops.down8(ws[0], g, xd, torch.from_numpy(hh).to(gpu), y, layout=LAYOUT_TILED)
    ops.iq3_gemv(ws[0], g, xd, o, layout=LAYOUT_TILED)
    outs = [torch.full((M, n), float("nan"), dtype=torch.float16, device=gpu) for n in ns]
    ops.iq3_gemv_multi(ws, g, xd, outs, layout=LAYOUT_TILED)
    torch.cuda.synchronize()
    refs = [gemv.gemv16_ref(quants.dequant_iq3xxs_packed(p, K), x)[1] for p in packed]
    _, yref = gemv.down8_ref(quants.dequant_iq3xxs_packed(packed[0], K), x, hh)
    ey, eo = _rows_err(y.cpu().numpy(), yref), _rows_err(o.cpu().numpy(), refs[0])
    print(f"[N=8200 down8] rel-err {ey:.3e}; [iq3_gemv] {eo:.3e}")
    assert ey <= TOL and eo <= TOL
    for n, out, ref in zip(ns, outs, refs):
        err = _rows_err(out.cpu().numpy(), ref)
        print(f"[multi N={n}] rel-err {err:.3e}")
        assert err <= TOL


def test_ffn8_hh_tiled_equals_two_calls(gpu):
    print("[case] ffn8_hh tiled M=11", flush=True)
    rng = synth.config_rng(6)
    M, N, K = 11, 256, 5120
    _, tg = _mat(gpu, rng, N, K)
    _, tu = _mat(gpu, rng, N, K)
    g = formats.gridf_tensor(gpu)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(gpu)
    ao = torch.from_numpy(synth.activations_f16(rng, M, K)).to(gpu)
    nw = torch.from_numpy((1 + 0.1 * rng.standard_normal(K)).astype(np.float32)).to(gpu)
    hh = torch.empty(M, K, device=gpu)
    hhx = torch.empty(M, K, dtype=torch.float16, device=gpu)
    fused = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.ffn8_hh(tg, tu, g, x, ao, nw, hh, hhx, fused, layout=LAYOUT_TILED)
    hh2, hhx2 = torch.empty_like(hh), torch.empty_like(hhx)
    sep = torch.empty_like(fused)
    ops.add_rms_f16(x, ao, nw, hh2, hhx2)
    ops.ffn8(tg, tu, g, hhx2, sep, layout=LAYOUT_TILED)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), sep.view(torch.int16))


def test_tiled_rejects_short_or_misaligned_buffers(gpu):
    N, K = 20, 256                                  # two tiles: 32 rows of records
    w = torch.zeros(20 * 98, dtype=torch.uint8, device=gpu)
    x = torch.zeros(1, K, dtype=torch.float16, device=gpu)
    out = torch.empty(1, N, dtype=torch.float16, device=gpu)
    g = formats.gridf_tensor(gpu)
    with pytest.raises(ValueError):
        ops.iq3_gemv(w, g, x, out, layout=LAYOUT_TILED)     # 20 rows of bytes, 32 needed
    big = torch.zeros(32 * 102 + 16, dtype=torch.uint8, device=gpu)
    with pytest.raises(TlxError):
        ops.iq3_gemv(big[8:], g, x, out, layout=LAYOUT_TILED)
    with pytest.raises(ValueError):                 # five matrices: one launch takes at most four
        ops.iq3_gemv_multi([big] * 5, g, x, [out] * 5, layout=LAYOUT_TILED)


@pytest.mark.parametrize("M", [1, 11])
@pytest.mark.parametrize("tiled", [True, False])
def test_multi_matrix_parity(gpu, M, tiled):
    """Four matrices sharing x in one launch (the GDN projections' shape pattern: a large, a
    medium and two 48-row matrices) against the oracle; tiled calls are deterministic."""
    print(f"[case] iq3_gemv_multi M={M} tiled={tiled}", flush=True)
    rng = synth.config_rng(7)
    K, ns = 5120, (1000, 600, 48, 48)
    packed = [formats.iq3_pack_rows(synth.iq3xxs_raw(rng, n, K), K) for n in ns]
    ws = [torch.from_numpy(p).to(gpu) for p in packed]
    lay = LAYOUT_TILED if tiled else LAYOUT_PACKED
    if tiled:
        ws = [_tiled(gpu, w, n, K) for w, n in zip(ws, ns)]
    x = synth.activations_f16(rng, M, K)
    xd = torch.from_numpy(x).to(gpu)
    g = formats.gridf_tensor(gpu)
    outs = [torch.full((M, n), float("nan"), dtype=torch.float16, device=gpu) for n in ns]
    ops.iq3_gemv_multi(ws, g, xd, outs, layout=lay)
    again = [torch.empty_like(o) for o in outs]
    ops.iq3_gemv_multi(ws, g, xd, again, layout=lay)
    torch.cuda.synchronize()
    for p, o, o2 in zip(packed, outs, again):
        _, ref = gemv.gemv16_ref(quants.dequant_iq3xxs_packed(p, K), x)
        err = _rows_err(o.cpu().numpy(), ref)
        print(f"[multi M={M} tiled={tiled} N={p.shape[0]}] rel-err {err:.3e}")
        assert err <= TOL
        assert torch.equal(o.view(torch.int16), o2.view(torch.int16))


def test_aq3k8_tiled_parity(gpu):
    print("[case] aq3k8 tiled M=11", flush=True)
    rng = synth.config_rng(8)
    M, K, Nq, Nk, Nv = 11, 5120, 768, 128, 128
    pq, tq = _mat(gpu, rng, Nq, K)
    pk, tk = _mat(gpu, rng, Nk, K)
    pv, tv = _mat(gpu, rng, Nv, K)
    x = synth.activations_f16(rng, M, K)
    q = torch.empty(M, Nq, dtype=torch.float16, device=gpu)
    k = torch.empty(M, Nk, dtype=torch.float16, device=gpu)
    v = torch.empty(M, Nv, dtype=torch.float16, device=gpu)
    ops.aq3k8(tq, tk, tv, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), q, k, v, layout=LAYOUT_TILED)
    torch.cuda.synchronize()
    for p, o in ((pq, q), (pk, k), (pv, v)):
        _, ref = gemv.gemv16_ref(quants.dequant_iq3xxs_packed(p, K), x)
        assert _rows_err(o.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("N,K,M", [(16, 256, 1), (20, 256, 4), (100, 512, 3), (300, 1024, 16), (64, 17408, 4)])
def test_tiled_small_and_unstaged_shapes(gpu, N, K, M):
    """Shapes with fewer records than waves (1- and 4-wave workgroups), a tail tile, M = 16 (the
    tile-ordered copy) and M = 4 at K = 17408 (activations read from memory, too large to stage)."""
    print(f"[case] iq3_gemv tiled N={N} K={K} M={M}", flush=True)
    rng = synth.config_rng(9)
    p, t = _mat(gpu, rng, N, K)
    x = synth.activations_f16(rng, M, K)
    o = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
    ops.iq3_gemv(t, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), o, layout=LAYOUT_TILED)
    torch.cuda.synchronize()
    _, ref = gemv.gemv16_ref(quants.dequant_iq3xxs_packed(p, K), x)
    err = _rows_err(o.cpu().numpy(), ref)
    print(f"[tiled small N={N} K={K} M={M}] rel-err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("M", [1, 4, 11, 16])
def test_tileord_handoff_ffn8_down8(gpu, M):
    """ffn8 writing its output in the tile-ordered form (TLX_OUT_TILEORD) and down8 reading it
    (TLX_IN_TILEORD) give the row-major calls' results bit for bit; the tile-ordered buffer holds
    the row-major rows and repeats row M-1 in slots M..15.  Shapes of config 2/3's FFN block."""
    print(f"[case] tile-ordered ffn8 -> down8 M={M} N=17408 K=5120", flush=True)
    rng = synth.config_rng(3)
    H, F = 5120, 17408
    _, tg = _mat(gpu, rng, F, H)
    _, tu = _mat(gpu, rng, F, H)
    _, td = _mat(gpu, rng, H, F)
    g = formats.gridf_tensor(gpu)
    x = torch.from_numpy(synth.activations_f16(rng, M, H)).to(gpu)
    hh = torch.randn(M, H, device=gpu)
    gact = torch.empty(M, F, dtype=torch.float16, device=gpu)
    ops.ffn8(tg, tu, g, x, gact, LAYOUT_TILED)
    gt = ops.tileord_empty(F, gpu)
    ops.ffn8(tg, tu, g, x, gt, LAYOUT_TILED, out_tileord=True)
    y = torch.empty(M, H, device=gpu)
    ops.down8(td, g, gact, hh, y, LAYOUT_TILED)
    yt = torch.empty(M, H, device=gpu)
    ops.down8(td, g, gt, hh, yt, LAYOUT_TILED, in_tileord=True)
    # the plain GEMV form over the same hand-off (fp16 output, tile-ordered both ways)
    o = torch.empty(M, H, dtype=torch.float16, device=gpu)
    ops.iq3_gemv(td, g, gact, o, LAYOUT_TILED)
    ot = ops.tileord_empty(H, gpu)
    ops.iq3_gemv(td, g, gt, ot, LAYOUT_TILED, in_tileord=True, out_tileord=True, m=M)
    torch.cuda.synchronize()
    rows = ops.tileord_to_rows(gt, 16).cpu().numpy()
    assert np.array_equal(rows[:M], gact.cpu().numpy())
    assert all(np.array_equal(rows[m], rows[M - 1]) for m in range(M, 16))
    assert np.array_equal(yt.cpu().numpy(), y.cpu().numpy())
    assert np.array_equal(ops.tileord_to_rows(ot, M).cpu().numpy(), o.cpu().numpy())


def test_tileord_flags_rejected(gpu):
    """The tile-ordered output exists for the tiled records only, and down8 has no fp16 output."""
    print("[case] tile-ordered flag checks", flush=True)
    from thunderllamax_amd import _lib
    rng = synth.config_rng(3)
    pg, tg = _mat(gpu, rng, 64, 512)
    g = formats.gridf_tensor(gpu)
    x = torch.from_numpy(synth.activations_f16(rng, 2, 512)).to(gpu)
    dp = torch.from_numpy(pg).to(gpu)
    with pytest.raises(TlxError):
        ops.ffn8(dp, dp, g, x, ops.tileord_empty(64, gpu), LAYOUT_PACKED, out_tileord=True)
    with pytest.raises(TlxError):
        _lib.call("tlx_down8", tg.data_ptr(), g.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(), 2, 64, 512,
                  LAYOUT_TILED | _lib.OUT_TILEORD, None)
