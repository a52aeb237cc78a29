"""Full-size shapes of the measured configurations that the unit-shape tests do not reach, and an
element-wise check of the fp16 SwiGLU epilogue.

* Config 4 at M = 8192: the prefill GEMMs (gate+up+SwiGLU, down+residual) at full K and N,
  checked on seeded weight-row samples over every activation row (norm-wise rel-err 1e-3 per
  row, as the other GEMM tests).
* Config 3's decode-step calls exactly as the benchmark makes them: the tiled out-projection
  5120 x 6144 at M = 11 (its activations do not fit the LDS stage: the tile-ordered copy path),
  the four GDN projections with their real row counts 10240 / 6144 / 48 / 48 in one launch, the
  raw Q6_K head 151936 x 5120 at M = 11, and aq6k8 with a raw Q6_K q and IQ3_XXS k / v rows.
* Tiled GEMVs of more than 2048 tiles (N > 32768 rows), which run as several launches with
  offset records, outputs and residuals.
* The SwiGLU epilogue element by element: ffn8's output equals swiglu16(half(ag), half(au))
  computed by the oracle from the GPU's own fp16 gate and up values (the plain GEMV over the same
  matrix sums the same products in the same order), within 1 fp16 ulp (the device exp2 and
  reciprocal against the oracle's correctly rounded ones).
"""
import numpy as np
import pytest
import torch

from oracle import gemv, quants
from thunderllamax_amd import formats, ops, synth
from thunderllamax_amd._lib import LAYOUT_PACKED, LAYOUT_RAW, LAYOUT_TILED

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _rows_err(y, ref):
    return max(gemv.rel_err(y[m], ref[m]) for m in range(ref.shape[0]))


def _tiled(gpu, packed, N, K):
    t = torch.empty(-(-N // 16) * 16 * 102 * (K // 256), dtype=torch.uint8, device=gpu)
    ops.pack_iq3_tiled(torch.from_numpy(packed).to(gpu), t, N, K)
    return t


def _iq3(rng, rows, kdim):
    return formats.iq3_pack_rows(synth.iq3xxs_raw(rng, rows, kdim), kdim)


def _ulp16(v):
    """fp16 ulp at |v| (normal range; subnormal spacing below 2^-14)."""
    a = np.maximum(np.abs(np.asarray(v, dtype=np.float64)), 2.0 ** -14)
    return 2.0 ** (np.floor(np.log2(a)) - 10)


# ------------------------------------------------------------------ config 4 at M = 8192
def test_pfg3_ffn_m8192_sampled_rows(gpu):
    print("[case] pfg3_ffn M=8192 K=5120 N=17408", flush=True)
    rng = synth.config_rng(4)
    M, N, K = 8192, 17408, 5120
    pg, pu = _iq3(rng, N, K), _iq3(rng, N, K)
    wg = torch.from_numpy(formats.iq3_pack7(pg, K)).to(gpu)
    wu = torch.from_numpy(formats.iq3_pack7(pu, K)).to(gpu)
    x = synth.activations_f16(rng, M, K)
    out = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.pfg3_ffn(wg, wu, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), out)
    torch.cuda.synchronize()
    cols = np.sort(np.random.default_rng(11).choice(N, 96, replace=False))
    _, _, ref = gemv.pf_ffn_ref(quants.dequant_iq3xxs_packed(pg[cols], K),
                                quants.dequant_iq3xxs_packed(pu[cols], K), x)
    y = out[:, torch.from_numpy(cols).to(gpu)].cpu().numpy()
    err = _rows_err(y, ref)
    print(f"[pfg3_ffn M=8192] sampled max row rel-err {err:.3e}")
    assert err <= TOL
    assert torch.isfinite(out.float()).all()


def test_pfg3_iq3d_m8192_sampled_rows(gpu):
    print("[case] pfg3_iq3d M=8192 K=17408 N=5120", flush=True)
    rng = synth.config_rng(4)
    M, N, K = 8192, 5120, 17408
    pw = _iq3(rng, N, K)
    w = torch.from_numpy(formats.iq3_pack7(pw, K)).to(gpu)
    x = synth.activations_f16(rng, M, K)
    res = rng.standard_normal((M, N)).astype(np.float32)
    out = torch.empty(M, N, dtype=torch.float32, device=gpu)
    ops.pfg3_iq3d(w, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), torch.from_numpy(res).to(gpu), out)
    torch.cuda.synchronize()
    cols = np.sort(np.random.default_rng(12).choice(N, 48, replace=False))
    acc, _ = gemv.pf_res_ref(quants.dequant_iq3xxs_packed(pw[cols], K), x, res[:, cols])
    y = out[:, torch.from_numpy(cols).to(gpu)].cpu().numpy()
    err = _rows_err(y.astype(np.float64) - res[:, cols], acc)
    print(f"[pfg3_iq3d M=8192] sampled max row rel-err (product) {err:.3e}")
    assert err <= TOL


# ------------------------------------------------------------------ config 3 call shapes
def test_outproj_tiled_5120x6144_m11(gpu):
    """The attention / GDN out-projection of the decode step: K = 6144 activations at M = 11 are
    too large for the LDS stage, so the tile-ordered copy path runs."""
    print("[case] iq3_gemv tiled 5120x6144 M=11", flush=True)
    rng = synth.config_rng(3)
    N, K, M = 5120, 6144, 11
    p = _iq3(rng, N, K)
    t = _tiled(gpu, p, N, K)
    x = synth.activations_f16(rng, M, K)
    o = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
    ops.iq3_gemv(t, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), o, layout=LAYOUT_TILED)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(13).choice(N, 512, replace=False))
    _, ref = gemv.gemv16_ref(quants.dequant_iq3xxs_packed(p[rows], K), x)
    err = _rows_err(o.cpu().numpy()[:, rows], ref)
    print(f"[out-proj tiled] sampled max row rel-err {err:.3e}")
    assert err <= TOL and torch.isfinite(o.float()).all()


@pytest.mark.parametrize("tiled", [True, False])
def test_gdn_projections_real_rows_m11(gpu, tiled):
    print(f"[case] iq3_gemv_multi 10240/6144/48/48 M=11 tiled={tiled}", flush=True)
    rng = synth.config_rng(3)
    K, M, ns = 5120, 11, (10240, 6144, 48, 48)
    packed = [_iq3(rng, n, K) for n in ns]
    if tiled:
        ws = [_tiled(gpu, p, n, K) for p, n in zip(packed, ns)]
    else:
        ws = [torch.from_numpy(p).to(gpu) for p in packed]
    x = synth.activations_f16(rng, M, K)
    outs = [torch.full((M, n), float("nan"), dtype=torch.float16, device=gpu) for n in ns]
    ops.iq3_gemv_multi(ws, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), outs,
                       layout=LAYOUT_TILED if tiled else LAYOUT_PACKED)
    torch.cuda.synchronize()
    srng = np.random.default_rng(14)
    for p, n, o in zip(packed, ns, outs):
        rows = np.arange(n) if n <= 256 else np.sort(srng.choice(n, 256, replace=False))
        _, ref = gemv.gemv16_ref(quants.dequant_iq3xxs_packed(p[rows], K), x)
        err = _rows_err(o.cpu().numpy()[:, rows], ref)
        print(f"[gdn N={n} tiled={tiled}] rel-err {err:.3e}")
        assert err <= TOL and torch.isfinite(o.float()).all()


def test_q6k_head_raw_151936_m11(gpu):
    print("[case] q6k_gemv16 raw 151936x5120 M=11", flush=True)
    rng = synth.config_rng(3)
    N, K, M = 151936, 5120, 11
    raw = synth.q6k_raw(rng, N, K)
    w = torch.from_numpy(raw).to(gpu)
    x = synth.activations_f16(rng, M, K)
    o = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
    ops.q6k_gemv16(w, torch.from_numpy(x).to(gpu), o, LAYOUT_RAW)
    torch.cuda.synchronize()
    rows = np.sort(np.concatenate([np.random.default_rng(15).choice(N - 64, 448, replace=False),
                                   np.arange(N - 64, N)]))   # the last tiles included
    _, ref = gemv.gemv16_ref(quants.dequant_q6k(raw[rows], K), x)
    err = _rows_err(o.cpu().numpy()[:, rows], ref)
    print(f"[q6k head raw] sampled max row rel-err {err:.3e}")
    assert err <= TOL and torch.isfinite(o.float()).all()


def test_aq6k8_raw_q_iq3_v_as_the_sweep_calls_it(gpu):
    """aq6k8 with a raw 210-B Q6_K q (12288 rows) and IQ3_XXS packed-row k and v (1024 rows
    each): the decode step's call on the Q6_K attention layers."""
    print("[case] aq6k8 raw q + IQ3 v M=11", flush=True)
    rng = synth.config_rng(3)
    M, K, Nq, Nk, Nv = 11, 5120, 12288, 1024, 1024
    rawq = synth.q6k_raw(rng, Nq, K)
    pk, pv = _iq3(rng, Nk, K), _iq3(rng, Nv, K)
    x = synth.activations_f16(rng, M, K)
    outs = [torch.full((M, n), float("nan"), dtype=torch.float16, device=gpu) for n in (Nq, Nk, Nv)]
    ops.aq6k8(torch.from_numpy(rawq).to(gpu), torch.from_numpy(pk).to(gpu), torch.from_numpy(pv).to(gpu),
              formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), *outs, layout=LAYOUT_RAW)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(16).choice(Nq, 384, replace=False))
    checks = [(outs[0], rows, quants.dequant_q6k(rawq[rows], K)),
              (outs[1], np.arange(Nk), quants.dequant_iq3xxs_packed(pk, K)),
              (outs[2], np.arange(Nv), quants.dequant_iq3xxs_packed(pv, K))]
    for o, r, W in checks:
        _, ref = gemv.gemv16_ref(W, x)
        err = _rows_err(o.cpu().numpy()[:, r], ref)
        print(f"[aq6k8 raw] rel-err {err:.3e}")
        assert err <= TOL


# ------------------------------------------------------------------ several tiled launches
def test_tiled_more_than_2048_tiles(gpu):
    """N = 33000 rows = 2063 tiles: the tiled GEMVs run a launch of 2048 tiles and one of 15, with
    record, output and residual offsets; plain, residual and SwiGLU forms against the oracle."""
    print("[case] tiled N=33000 K=256 (two launches)", flush=True)
    rng = synth.config_rng(10)
    N, K, M = 33000, 256, 3
    pa, pb = _iq3(rng, N, K), _iq3(rng, N, K)
    ta, tb = _tiled(gpu, pa, N, K), _tiled(gpu, pb, N, K)
    g = formats.gridf_tensor(gpu)
    x = synth.activations_f16(rng, M, K)
    xd = torch.from_numpy(x).to(gpu)
    hh = rng.standard_normal((M, N)).astype(np.float32)
    o = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
    y = torch.full((M, N), float("nan"), device=gpu)
    f = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
    ops.iq3_gemv(ta, g, xd, o, layout=LAYOUT_TILED)
    ops.down8(ta, g, xd, torch.from_numpy(hh).to(gpu), y, layout=LAYOUT_TILED)
    ops.ffn8(ta, tb, g, xd, f, layout=LAYOUT_TILED)
    torch.cuda.synchronize()
    Wa, Wb = quants.dequant_iq3xxs_packed(pa, K), quants.dequant_iq3xxs_packed(pb, K)
    _, oref = gemv.gemv16_ref(Wa, x)
    _, yref = gemv.down8_ref(Wa, x, hh)
    _, _, fref = gemv.ffn8_ref(Wa, Wb, x)
    for name, got, ref in (("iq3_gemv", o, oref), ("down8", y, yref), ("ffn8", f, fref)):
        err = _rows_err(got.cpu().numpy(), ref)
        tail = _rows_err(got.cpu().numpy()[:, 32768:], ref[:, 32768:])
        print(f"[{name} N=33000] rel-err {err:.3e}, rows past the first launch {tail:.3e}")
        assert err <= TOL and tail <= TOL
    # the tile-ordered outputs of both launches (the second starts at column group 4096)
    ot = ops.tileord_empty(N, gpu)
    ft = ops.tileord_empty(N, gpu)
    ops.iq3_gemv(ta, g, xd, ot, layout=LAYOUT_TILED, out_tileord=True)
    ops.ffn8(ta, tb, g, xd, ft, layout=LAYOUT_TILED, out_tileord=True)
    torch.cuda.synchronize()
    assert np.array_equal(ops.tileord_to_rows(ot, M).cpu().numpy(), o.cpu().numpy())
    assert np.array_equal(ops.tileord_to_rows(ft, M).cpu().numpy(), f.cpu().numpy())


# ------------------------------------------------------------------ the SwiGLU epilogue
@pytest.mark.parametrize("layout", [LAYOUT_TILED, LAYOUT_PACKED])
def test_ffn8_epilogue_elementwise(gpu, layout):
    print(f"[case] ffn8 epilogue element-wise layout={layout}", flush=True)
    rng = synth.config_rng(2)
    N, K, M = 1000, 5120, 11
    pg, pu = _iq3(rng, N, K), _iq3(rng, N, K)
    if layout == LAYOUT_TILED:
        wg, wu = _tiled(gpu, pg, N, K), _tiled(gpu, pu, N, K)
    else:
        wg, wu = torch.from_numpy(pg).to(gpu), torch.from_numpy(pu).to(gpu)
    g = formats.gridf_tensor(gpu)
    xd = torch.from_numpy(synth.activations_f16(rng, M, K)).to(gpu)
    act = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ag = torch.empty_like(act)
    au = torch.empty_like(act)
    ops.ffn8(wg, wu, g, xd, act, layout=layout)
    ops.iq3_gemv(wg, g, xd, ag, layout=layout)
    ops.iq3_gemv(wu, g, xd, au, layout=layout)
    torch.cuda.synchronize()
    want = gemv.swiglu16(ag.cpu().numpy(), au.cpu().numpy()).astype(np.float64)
    got = act.cpu().numpy().astype(np.float64)
    d = np.abs(got - want)
    ulps = d / _ulp16(want)
    print(f"[ffn8 epilogue layout={layout}] max {ulps.max():.2f} ulp, "
          f"{int((d > 0).sum())} of {d.size} elements differ")
    assert np.isfinite(got).all()
    assert (ulps <= 1.0).all()
